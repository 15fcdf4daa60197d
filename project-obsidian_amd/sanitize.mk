# sanitize.mk — the checkpoint reader's host-sanitizer checker
# (tests/loader_check.cpp, run by tests/test_loader_sanitized.py):
#   make -f sanitize.mk
# Every source's host code is built with AddressSanitizer and UBSan (each flag
# after -Xarch_host, so the GPU code is built as the main Makefile builds it)
# and linked with the checker by clang++. Nothing here is part of the library.
HIPCC ?= /opt/rocm/bin/hipcc
CLANGXX ?= /opt/rocm/llvm/bin/clang++
ARCH ?= gfx950
HIPFLAGS ?= -O3 -std=c++17 -fPIC --offload-arch=$(ARCH) -ffp-contract=off \
            -Xclang -target-feature -Xclang -packed-fp32-ops -Wall -Wno-unused-result
SANFLAGS := -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined \
            -Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer
SRCS := $(wildcard csrc/*.hip)
SAN_OBJS := $(patsubst csrc/%.hip,_build_san/%.o,$(SRCS))

_build_san/loader_check: $(SAN_OBJS) ../tests/loader_check.cpp
	$(CLANGXX) -O1 -g -fsanitize=address,undefined -fno-sanitize-recover=undefined -I ../include \
	    -o $@ ../tests/loader_check.cpp $(SAN_OBJS) -L/opt/rocm/lib -lamdhip64 -Wl,-rpath,/opt/rocm/lib

_build_san/%.o: csrc/%.hip csrc/obs_internal.hpp ../include/obsidian_hip.h
	@mkdir -p _build_san
	$(HIPCC) $(HIPFLAGS) $(SANFLAGS) -c $< -o $@
