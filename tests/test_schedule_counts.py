"""The refill schedule's word count in closed form.

csrc/encode.hip counts the stream words each lane takes from two bit totals
(up to the third- and second-to-last segments) instead of replaying the
schedule.  This checks that closed form against a step-by-step replay of the
decoders' rule on random bit counts, including zero-bit steps, step counts
that end inside a segment, and the largest steps.  The rule: two words to
start; the steps are cut into segments (step pairs with 2^12-state tables,
nb <= 12; 3, 3 and 2 steps of every 8 with 2^11-state tables, nb <= 10);
after every segment but the last a lane takes a word at <= 32 unread bits,
after the second-to-last only below what the last segment can read (24 for
pairs, 10 per step of the last segment otherwise) -- except when the last
16-element tile (8 pair steps, 16 steps of the 3-3-2 schedule) holds a
single segment: that check then follows the tile before and is the plain
one.  The GPU encoder's output is checked byte for byte against the CPU
encoder in tests/test_gpu_encode.py.
"""
import random

import pytest


def segments(S, triple):
    """(first, end) steps of each segment of S steps."""
    out, i = [], 0
    lens = (3, 3, 2) if triple else (2,)
    while i < S:
        for n in lens:
            if i >= S:
                break
            out.append((i, min(i + n, S)))
            i += n
    return out


def tile_steps(triple):
    return 16 if triple else 8


def final_below(segs, triple):
    a, b = segs[-1]
    ts = tile_steps(triple)
    if b > ts and a == ts * ((b - 1) // ts):   # the last tile holds one segment
        return 33
    return 10 * (b - a) if triple else 24


def replay(nbs, triple):
    """Words taken by one lane whose steps consume nbs[0], nbs[1], ... bits."""
    segs = segments(len(nbs), triple)
    if not segs:
        return 0
    taken, held = 2, 64
    for q, (a, b) in enumerate(segs):
        seg_bits = sum(nbs[a:b])
        assert seg_bits <= 30 if triple else seg_bits <= 24
        assert held >= 33 or q + 1 == len(segs) or q == 0, "at least 33 bits into a segment"
        held -= seg_bits
        assert held >= 0, "the schedule never lets a lane run dry"
        if q + 1 < len(segs):
            below = final_below(segs, triple) if q + 2 == len(segs) else 33
            if held < below:
                taken += 1
                held += 32
    return taken


def closed_form(nbs, triple):
    """The encoder's count: t = c3 // 32 + 2, plus one when 32 t - c2 is
    below the final threshold."""
    segs = segments(len(nbs), triple)
    n = len(segs)
    if n == 0:
        return 0
    if n == 1:
        return 2
    bits = sum(nbs)
    b1 = sum(nbs[segs[-1][0]:])          # the last segment
    b2 = sum(nbs[segs[-2][0]:])          # the last two segments
    c2 = bits - b1
    c3 = bits - b2 if n >= 3 else 0
    t = c3 // 32 + 2
    return t + (1 if 32 * t - c2 < final_below(segs, triple) else 0)


def max_words(S, triple, top_nb):
    """The most words one lane can take over S steps of at most top_nb bits
    each, over every way the bits can fall (the rule of replay(), by
    dynamic programming over the bits the lane holds)."""
    segs = segments(S, triple)
    states = {64: 2}   # bits held -> most words taken so far
    for q, (a, b) in enumerate(segs):
        nxt = {}
        for held, taken in states.items():
            for c in range(0, min(held, (b - a) * top_nb) + 1):
                h, t = held - c, taken
                if q + 1 < len(segs):
                    below = final_below(segs, triple) if q + 2 == len(segs) else 33
                    if h < below:
                        h, t = h + 32, t + 1
                nxt[h] = max(nxt.get(h, 0), t)
        states = nxt
    return max(states.values())


@pytest.mark.parametrize("triple,top_nb,ring_segments", [(False, 12, 1), (True, 10, 2)])
def test_one_tile_streams_fit_the_first_segments(triple, top_nb, ring_segments):
    """fused_add_kernel<..., FIRST = kOneTileSegs> loads a stream of one
    16-element tile whole at its start into that many ring segments of 256 words
    (1 for pairs, 2 for nibbles) and never fetches again: 64 lanes of at
    most 3 (pair) or 5 (nibble) words fit.  The DP agrees with replay() on
    the sequences that reach the bound."""
    worst = 0
    for S in range(1, tile_steps(triple) + 1):
        w = max_words(S, triple, top_nb)
        assert 64 * w <= 256 * ring_segments, (S, w)
        worst = max(worst, w)
    assert worst == (5 if triple else 3)
    S = tile_steps(triple)
    assert max(replay([top_nb] * S, triple), replay([0] * S, triple)) <= worst
    assert max_words(S, triple, top_nb) >= replay([top_nb] * S, triple)


@pytest.mark.parametrize("triple,top_nb,tiles", [(False, 12, 4), (True, 10, 2)])
def test_resident_streams_fit_the_ring(triple, top_nb, tiles):
    """fused_add_kernel<..., FIRST = kSlots> loads streams of up to
    Alpha::kResidentTiles tiles (4 for pairs, 2 for nibbles) whole into the
    ring's 3 segments of 256 words: 64 lanes of at most 12 words fit, and
    one more tile would not."""
    for S in range(1, tiles * tile_steps(triple) + 1):
        assert 64 * max_words(S, triple, top_nb) <= 3 * 256, S
    S = (tiles + 1) * tile_steps(triple)
    assert 64 * max_words(S, triple, top_nb) > 3 * 256


@pytest.mark.parametrize("triple,top_nb", [(False, 12), (True, 10)])
def test_closed_form_equals_replay(triple, top_nb):
    rng = random.Random(7)
    for _ in range(20000):
        S = rng.choice([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 14, 16, 31, 64, 257])
        top = rng.choice([0, 1, 2, 5, top_nb - 1, top_nb])
        nbs = [rng.randint(0, top) if rng.random() < 0.8 else top for _ in range(S)]
        assert closed_form(nbs, triple) == replay(nbs, triple), nbs


@pytest.mark.parametrize("triple,top_nb", [(False, 12), (True, 10)])
def test_closed_form_extremes(triple, top_nb):
    for S in range(0, 40):
        for v in (0, 1, top_nb - 1, top_nb):
            nbs = [v] * S
            assert closed_form(nbs, triple) == replay(nbs, triple), (S, v)


def test_segments_of_the_triple_schedule():
    assert segments(8, True) == [(0, 3), (3, 6), (6, 8)]
    assert segments(12, True) == [(0, 3), (3, 6), (6, 8), (8, 11), (11, 12)]
    assert segments(5, False) == [(0, 2), (2, 4), (4, 5)]


# ---------------------------------------------------------------------------
# Where the GPU decoders put the checks.  They decode 16-element tiles and
# run every tile but the last through a path whose checks are all the plain
# one; the last tile chooses per segment between the plain check, the final
# check and none.  libtans_amd.so exports the thresholds both sides apply
# (csrc/schedule.h: encoder_below, the rule csrc/codec.cpp encodes with, and
# decoder_below, what that placement amounts to), compared here for every
# stream length and with the rule as restated above.

def _check_below():
    import ctypes
    from rans_vectoradd._lib import lib
    fn = lib.tans_internal_check_below
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64]
    return fn


def restated_below(S, triple, j):
    segs = segments(S, triple)
    n = len(segs)
    return 0 if j + 1 >= n else final_below(segs, triple) if j + 2 == n else 33


def without_the_tile_rule(S, triple, j):
    """The final threshold as the last segment's reach alone: with it the
    check after segment n - 2 disagrees with the decoders' plain path
    whenever the last tile holds a single segment."""
    segs = segments(S, triple)
    n = len(segs)
    a, b = segs[-1]
    return 0 if j + 1 >= n else (10 * (b - a) if triple else 24) if j + 2 == n else 33


@pytest.mark.parametrize("triple", [False, True])
def test_decoder_check_placement_matches_the_encoders(triple):
    fn = _check_below()
    ts = tile_steps(triple)
    differs = set()
    for S in range(1, 12 * ts + 1):
        for j in range(len(segments(S, triple))):
            enc, dec = fn(0, S, int(triple), j), fn(1, S, int(triple), j)
            assert enc == dec == restated_below(S, triple, j), (S, j, enc, dec)
            if without_the_tile_rule(S, triple, j) != dec:
                differs.add(S % ts)
    # exactly the streams whose last tile holds one segment: pair streams of
    # 1 or 2 steps past whole tiles (N % 16 = 2 or 4, N > 16), 3-3-2 streams
    # of 1-3 steps (N % 16 = 1..3)
    assert differs == ({1, 2} if not triple else {1, 2, 3})
