// Refill schedule of a lane's decode steps, shared by the CPU encoder
// (codec.cpp), the GPU encoder (encode.hip) and the decoders (kernels.hip).
//
// A lane's S decode steps are cut into segments.  A decoder reads each
// segment's bits from one 32-bit window taken at the lane's bit position,
// and after every segment but the last it checks the refill: a lane holding
// at most 32 unread bits takes the next word of its group's stream (after
// the second-to-last segment: only a lane holding fewer than `final_below`
// bits, the most the last segment can read).  Every lane starts with two
// words, so a lane enters each segment with at least 33 unread bits.
//
// * Tables of 2^12 states (the pair alphabet, nb <= 12): segments of two
//   steps (at most 24 bits).
// * Tables of 2^11 states (the nibble alphabet): every present symbol has a
//   frequency of at least 2, so nb <= 10, and each 8 steps are cut into
//   segments of 3, 3 and 2 steps (at most 30 bits).  Three steps per window
//   and per check, against two, take 6 fewer VALU instructions per 8 steps.
#ifndef TANS_SCHEDULE_H
#define TANS_SCHEDULE_H

#include <stdint.h>

#ifdef __HIPCC__
#define TANS_SCHED_FN constexpr __host__ __device__ __forceinline__
#else
#define TANS_SCHED_FN constexpr
#endif

namespace tans_sched {

constexpr int kTripleLog2L = 11;    // tables of this size use 3-3-2 segments
constexpr uint32_t kTripleMinFreq = 2;   // ... and every present symbol needs f >= 2
constexpr uint32_t kTripleMaxNb = 10;
constexpr int kAtMost = 32;         // a lane holding at most this many bits takes a word
constexpr int kPairFinalBelow = 24; // pair schedule: the final check's threshold

// Segments of S steps.
TANS_SCHED_FN int64_t segments(int64_t S, bool triple) {
    if (!triple) return (S + 1) / 2;
    const int64_t r = S % 8;
    return 3 * (S / 8) + (r == 0 ? 0 : r <= 3 ? 1 : r <= 6 ? 2 : 3);
}

// First step of segment j.
TANS_SCHED_FN int64_t seg_start(int64_t j, bool triple) {
    if (!triple) return 2 * j;
    const int64_t w = j % 3;
    return 8 * (j / 3) + (w == 0 ? 0 : w == 1 ? 3 : 6);
}

// Steps in the last segment of S > 0 steps.
TANS_SCHED_FN int last_len(int64_t S, bool triple) {
    return (int)(S - seg_start(segments(S, triple) - 1, triple));
}

// Decode steps per 16-element tile (the sign/mantissa tile of the format):
// 8 pair steps, or 16 steps of the 3-3-2 schedule (two of its 8-step
// periods, so a tile boundary is always a segment boundary).
TANS_SCHED_FN int64_t tile_steps(bool triple) { return triple ? 16 : 8; }

// Segments in the last tile of a stream of S > 0 steps.
TANS_SCHED_FN int64_t last_tile_segments(int64_t S, bool triple) {
    const int64_t ts = tile_steps(triple);
    return segments(S - ts * ((S - 1) / ts), triple);
}

// The final check's threshold: the most bits the last segment can read.
// When the last tile holds a single segment, the final check follows the
// last segment of the tile before it; it is then the plain check (a word
// at kAtMost bits or fewer), so that the decoders run every tile but the
// last through one code path.
TANS_SCHED_FN int final_below(int64_t S, bool triple) {
    if (S > tile_steps(triple) && last_tile_segments(S, triple) == 1) return kAtMost + 1;
    return triple ? (int)kTripleMaxNb * last_len(S, triple) : kPairFinalBelow;
}

// The encoders' threshold after segment j of S steps: a lane holding fewer
// bits takes a word; 0 after the last segment (no check).
TANS_SCHED_FN int encoder_below(int64_t S, bool triple, int64_t j) {
    const int64_t n_seg = segments(S, triple);
    return j + 1 >= n_seg ? 0 : j + 2 == n_seg ? final_below(S, triple) : kAtMost + 1;
}

// How the decoders place the checks.  Every tile but the last takes the
// plain path (every check at kAtMost + 1); the last tile, starting with
// `segs` segments, puts the final check after its segment segs - 2 and
// none from segment segs - 1 on.
TANS_SCHED_FN bool end_is_final(int segs, int idx) { return idx == segs - 2; }
TANS_SCHED_FN bool end_is_none(int segs, int idx) { return idx >= segs - 1; }

// The decoders' threshold after segment j, from that placement (equal to
// encoder_below for every S and j).
TANS_SCHED_FN int decoder_below(int64_t S, bool triple, int64_t j) {
    const int64_t n_seg = segments(S, triple);
    const int64_t first = n_seg - last_tile_segments(S, triple);   // the last tile's first segment
    if (j < first) return kAtMost + 1;
    const int segs = (int)(n_seg - first), idx = (int)(j - first);
    return end_is_none(segs, idx) ? 0 : end_is_final(segs, idx) ? final_below(S, triple)
                                                                 : kAtMost + 1;
}

}  // namespace tans_sched

// The packed layout of short streams (pair alphabet, at most kMaxSteps
// steps per lane), shared by the CPU encoder and the decoders.  A group's
// stream is a header of kPairs lane-pair bit counts (hdr_bytes each) and a
// bit area right after it.  Lane pair p = lanes 2p, 2p + 1 owns bits
// [S_p, E_p) of the area, S_p = the counts of the pairs before it summed,
// E_p = S_p + count p.  A lane's bits in decode order are its initial
// state minus L (kStateBits) and then each step's nb bits, LSB first; the
// even lane's go forwards from S_p (its i-th bit at S_p + i), the odd
// lane's backwards from E_p (its i-th bit at E_p - 1 - i).  Bit b of the
// area is bit b % 8 of its byte b / 8.  No refill schedule: a decoder keeps
// one bit cursor per lane.  The stream is padded with zeros to 16 bytes.
namespace tans_pack {

constexpr int kPairs = 32;          // lane pairs of a 64-lane group
constexpr int kStateBits = 12;      // the state minus L, 2^12-state tables
constexpr int kMaxNb = 12;
constexpr int64_t kMaxSteps = 32;   // 64 elements per lane (four 16-element tiles)

// Header entry bytes: one while a pair's bits fit (8 steps: at most
// 2 * (12 + 8 * 12) = 216), else two.
TANS_SCHED_FN int hdr_bytes(int64_t S) { return S <= 8 ? 1 : 2; }
TANS_SCHED_FN int hdr_total(int64_t S) { return kPairs * hdr_bytes(S); }

// The most bits one lane can hold for S steps.
TANS_SCHED_FN int64_t max_lane_bits(int64_t S) { return kStateBits + (int64_t)kMaxNb * S; }

// The most bytes a group's stream can take (header, area, padding to 16).
TANS_SCHED_FN int64_t max_stream_bytes(int64_t S) {
    return (hdr_total(S) + (2 * kPairs * max_lane_bits(S) + 7) / 8 + 15) / 16 * 16;
}

}  // namespace tans_pack

#endif  // TANS_SCHEDULE_H
