// loader_check.cpp — drives the checkpoint reader (obs_ckpt_*) over a list of
// model directories, for the host-sanitizer test of the parser
// (test_loader_sanitized.py builds it with AddressSanitizer and UBSan).
//
// Input: one job per line, the model directory then the tensor names, each
// hex-encoded (names may hold tabs, quotes or any UTF-8), separated by spaces.
// Output: one line per job, the same fields as the test's ctypes rendering of
// the same calls: "open RC", then " config RC" (with the shape fields when RC
// is 0), then per name " | RC" (with dtype, shape, nbytes, the read's RC and
// an FNV-1a hash of the bytes when RC is 0).
#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "obsidian_hip.h"

namespace {

std::string unhex(const std::string& h) {
  std::string out;
  for (size_t i = 0; i + 1 < h.size(); i += 2) out.push_back(static_cast<char>(std::stoi(h.substr(i, 2), nullptr, 16)));
  return out;
}

uint64_t fnv1a(const unsigned char* p, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 0x100000001b3ull;
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s JOBS\n", argv[0]);
    return 2;
  }
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return 2;
  std::string line;
  for (int c; (c = std::fgetc(f)) != EOF;) {
    if (c != '\n') {
      line.push_back(static_cast<char>(c));
      continue;
    }
    std::vector<std::string> field;
    size_t a = 0;
    while (a < line.size()) {
      size_t b = line.find(' ', a);
      if (b == std::string::npos) b = line.size();
      field.push_back(unhex(line.substr(a, b - a)));
      a = b + 1;
    }
    line.clear();
    if (field.empty()) continue;
    obs_ckpt* ck = nullptr;
    const int rc = obs_ckpt_open(field[0].c_str(), nullptr, &ck);
    std::printf("open %d", rc);
    if (rc == OBS_OK) {
      obs_moe_config cfg;
      uint32_t n_layers = 0;
      const int rcc = obs_ckpt_config(ck, &cfg, &n_layers);
      std::printf(" config %d", rcc);
      if (rcc == OBS_OK)
        std::printf(" %u %u %u %u %u %u", cfg.n_exp, cfg.top_k, cfg.hidden, cfg.inter, cfg.group, n_layers);
      for (size_t i = 1; i < field.size(); ++i) {
        obs_tensor_info info;
        const int ri = obs_ckpt_tensor_info(ck, field[i].c_str(), &info);
        std::printf(" | %d", ri);
        if (ri != OBS_OK) continue;
        std::printf(" %d [", info.dtype);
        for (uint32_t d = 0; d < info.ndim && d < 8; ++d) std::printf(d ? ",%" PRIu64 : "%" PRIu64, info.shape[d]);
        std::printf("] %" PRIu64, info.nbytes);
        std::vector<unsigned char> buf(info.nbytes ? info.nbytes : 1);
        const int rr = obs_ckpt_read(ck, field[i].c_str(), buf.data(), info.nbytes);
        std::printf(" %d %016" PRIx64, rr, rr == OBS_OK ? fnv1a(buf.data(), info.nbytes) : uint64_t{0});
      }
      obs_ckpt_close(ck);
    }
    std::printf("\n");
  }
  std::fclose(f);
  return 0;
}
