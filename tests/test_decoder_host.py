"""Host logic of Model.run_turn (forward.rs:471-535) on the CPU: prefix reuse
against the cached tokens, the prompt's tail kept when it would overflow the
cache, batched or per-token prefill by suffix length, the positions each
token is fed at, and eos. The device calls are replaced by a recorder whose
'next token' is a fixed function of (token, position)."""
import pytest

import obsidian_hip as oh
from obsidian_hip import decoder as D

V = 1000


def nxt(tok, pos):
    return (tok * 31 + pos * 7 + 3) % V


class Rec(D.Model):
    def __init__(self, max_len):  # no device: only the host fields run_turn uses
        self.cfg = D.DecoderConfig(max_len=max_len)
        self.last_seq, self.last_reused, self.last_prefilled = [], 0, 0
        self.fail_prefill = False
        self.fed = {}      # position -> token whose keys/values it holds
        self.calls = []
        self._state = (0, 0)

    def prefill(self, tokens, pos0):
        self.calls.append(("prefill", pos0, len(tokens)))
        if self.fail_prefill:  # as a failing library call would, after writing part of the caches
            for i, t in enumerate(tokens[: len(tokens) // 2]):
                self.fed[pos0 + i] = -1
            raise oh.ObsError(oh.OBS_E_NOMEM, "obs_moe_prefill: workspace too small")
        for i, t in enumerate(tokens):
            self.fed[pos0 + i] = t
        self._state = (pos0 + len(tokens), nxt(tokens[-1], pos0 + len(tokens) - 1))
        return self._state[1]

    def fill_kv(self, tok, pos):
        self.calls.append(("fill", pos))
        self.fed[pos] = tok

    def run_one_token(self, tok, pos):
        self.calls.append(("one", pos))
        self.fed[pos] = tok
        self._state = (pos + 1, nxt(tok, pos))
        return self._state[1]

    def set_state(self, pos, tok):
        self._state = (pos, tok)

    def replay(self, n=1):
        pos, tok = self._state
        self.calls.append(("replay", pos))
        self.fed[pos] = tok
        self._state = (pos + 1, nxt(tok, pos))

    def read_state(self):
        return self._state


def expected(prompt, max_new, eos):
    gen = [nxt(prompt[-1], len(prompt) - 1)]
    pos = len(prompt)
    while len(gen) < max_new and gen[-1] != eos:
        gen.append(nxt(gen[-1], pos))
        pos += 1
    return gen


def test_first_turn_batched_and_per_token():
    m = Rec(4096)
    p = list(range(10, 40))
    assert m.run_turn(p, 5, eos=-1) == expected(p, 5, -1)
    assert m.calls[0] == ("prefill", 0, 30) and (m.last_reused, m.last_prefilled) == (0, 30)
    m2 = Rec(4096)
    p = [1, 2, 3]
    assert m2.run_turn(p, 2, eos=-1) == expected(p, 2, -1)
    assert m2.calls[:3] == [("fill", 0), ("fill", 1), ("one", 2)]


def test_prefix_reuse_covers_only_fed_tokens():
    m = Rec(4096)
    p1 = list(range(50, 80))
    g1 = m.run_turn(p1, 4, eos=-1)
    assert m.last_seq == p1 + g1[:-1]
    assert all(m.fed[i] == t for i, t in enumerate(m.last_seq))
    p2 = p1 + g1 + [5, 6]
    m.calls.clear()
    g2 = m.run_turn(p2, 3, eos=-1)
    assert (m.last_reused, m.last_prefilled) == (len(p1) + len(g1) - 1, 3)
    assert m.calls[:3] == [("fill", 33), ("fill", 34), ("one", 35)]
    assert g2 == expected(p2, 3, -1)
    assert all(m.fed[i] == t for i, t in enumerate(m.last_seq))


def test_identical_prompt_keeps_the_last_token_to_recompute():
    m = Rec(4096)
    p = list(range(30))
    m.run_turn(p, 1, eos=-1)          # caches hold p (max_new 1: nothing generated is fed)
    m.calls.clear()
    m.run_turn(p, 1, eos=-1)
    assert (m.last_reused, m.last_prefilled) == (29, 1) and m.calls == [("one", 29)]


def test_eos_stops_generation():
    m = Rec(4096)
    p = [4, 5, 6]
    first = nxt(6, 2)
    assert m.run_turn(p, 10, eos=first) == [first]
    full = expected(p, 6, -1)
    m2 = Rec(4096)
    assert m2.run_turn(p, 6, eos=full[2]) == full[:3]


def test_overflowing_prompt_keeps_its_tail():
    m = Rec(64)
    p = list(range(100))
    g = m.run_turn(p, 10, eos=-1)
    kept = p[100 - (64 - 11):]
    assert m.calls[0] == ("prefill", 0, len(kept)) and g == expected(kept, 10, -1)
    assert max(m.fed) < 64
    with pytest.raises(ValueError, match="no room"):
        Rec(8).run_turn([1, 2], 8, eos=-1)


def test_failed_batched_prefill_falls_back_to_token_steps(monkeypatch):
    """forward.rs:497-507: a batched prefill that fails is redone token by
    token from the reused prefix (the same positions, rewritten), and the
    turn's tokens are those of the per-token path."""
    m = Rec(4096)
    m.fail_prefill = True
    p = list(range(200, 240))
    g = m.run_turn(p, 3, eos=-1)
    assert g == expected(p, 3, -1) and "workspace" in m.last_fallback
    assert m.calls[0] == ("prefill", 0, 40) and m.calls[1:40] == [("fill", i) for i in range(39)]
    assert m.calls[40] == ("one", 39)
    assert all(m.fed[i] == t for i, t in enumerate(m.last_seq))
    m2 = Rec(4096)
    monkeypatch.setenv("OBSIDIAN_NO_BATCH", "1")  # the reference's switch: per-token only
    assert m2.run_turn(p, 2, eos=-1) == expected(p, 2, -1) and m2.calls[0] == ("fill", 0)
    assert m2.last_fallback is None
