"""The refill schedule's word count in closed form.

csrc/encode.hip counts the stream words each lane takes from two bit totals
(up to the third- and second-to-last step pairs) instead of replaying the
schedule.  This checks that closed form against a step-by-step replay of the
decoders' rule (two words to start; after every step pair but the last, take
a word at <= 32 unread bits; after the second-to-last, below 24) on random
bit counts, including zero-bit steps, odd step counts and the largest step
(12 bits, pair alphabet).  The GPU encoder's output is checked byte for byte
against the CPU encoder in tests/test_gpu_encode.py.
"""
import random


def replay(nbs):
    """Words taken by one lane whose steps consume nbs[0], nbs[1], ... bits."""
    S = len(nbs)
    if S == 0:
        return 0
    n_pairs = (S + 1) // 2
    taken, held = 2, 64
    for q in range(n_pairs):
        held -= sum(nbs[2 * q:2 * q + 2])
        assert held >= 0, "the schedule never lets a lane run dry"
        if q + 1 < n_pairs:
            below = 24 if q + 2 == n_pairs else 33
            if held < below:
                taken += 1
                held += 32
    return taken


def closed_form(nbs):
    """The encoder's count: t = c3 // 32 + 2, plus one when 32 t - c2 < 24."""
    S = len(nbs)
    if S == 0:
        return 0
    n = (S + 1) // 2
    if n == 1:
        return 2
    bits = sum(nbs)
    b1 = sum(nbs[2 * (n - 1):])          # the last pair
    b2 = sum(nbs[2 * (n - 2):])          # the last two pairs
    c2 = bits - b1
    c3 = bits - b2 if n >= 3 else 0
    t = c3 // 32 + 2
    return t + (1 if 32 * t - c2 < 24 else 0)


def test_closed_form_equals_replay():
    rng = random.Random(7)
    for _ in range(20000):
        S = rng.choice([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 16, 31, 64, 257])
        top = rng.choice([0, 1, 2, 5, 11, 12])
        nbs = [rng.randint(0, top) if rng.random() < 0.8 else top for _ in range(S)]
        assert closed_form(nbs) == replay(nbs), nbs


def test_closed_form_extremes():
    for S in range(0, 40):
        for v in (0, 1, 11, 12):
            nbs = [v] * S
            assert closed_form(nbs) == replay(nbs), (S, v)
