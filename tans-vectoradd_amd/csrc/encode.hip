// gfx950 tANS encoder into the wave64 lane layout (include/tans_amd.h).
// It writes the same bytes as the CPU encoder in codec.cpp: the same
// backward tANS construction (csrc/tans_codec.cpp:22-60 of the reference:
// walk the symbols backwards from x = L, emit the low nb bits that bring x
// into [f_s, 2 f_s), then x = L + slot of the rank-th occurrence of s), the
// same per-step bit chunks written forwards LSB-first, and the same refill
// schedule ordering the words of a group's 64 lanes.
//
// Passes (all on the caller's stream):
//   enc_backward_kernel  one thread per lane: step chunks [S][K] (u16:
//                        value in bits 11:0, nb in bits 15:12), the
//                        initial decoder state, and the number of stream
//                        words the lane takes (a closed form of the refill
//                        schedule in the lane's bit counts), summed per
//                        group (padded to 4); for rows of whole 16-byte
//                        tiles also the sign/mantissa tiles
//   enc_scan_kernel      exclusive prefix of the group counts -> offsets
//   enc_place_kernel     one wave per group: replays the schedule while
//                        each lane packs its chunks into words; a word's
//                        place (offset + handed + rank) is fixed when the
//                        lane takes it, and the word is stored there when
//                        its last bit is packed
//   enc_sm_kernel        sign/mantissa tiles when rows are not whole tiles
//
// The packed layout of short streams (pair alphabet, at most 32 steps per
// lane; schedule.h, tans_pack) reuses the backward pass, which then records
// each lane's bit count and state in the workspace and sums the group's
// bits into its stream size; enc_place_packed_kernel assembles each group's
// stream (header of lane-pair counts, bit area) in LDS and copies it out.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <type_traits>

#include "../../include/tans_amd.h"
#include "schedule.h"

extern "C" void tans_internal_set_error(const char* msg);  // codec.cpp

namespace {

constexpr int kLanes = 64;
constexpr int kTile = 16;
constexpr int64_t kTailWords = 256;
constexpr int kEncBlock = 256;

int fail(int code, const std::string& msg) {
    tans_internal_set_error(msg.c_str());
    return code;
}

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return TANS_OK;
    return fail(TANS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Workspace layout: chunks u16 [S][K], glen u32 [G].
struct WsLayout {
    int64_t chunks, glen, plen, pstate, total;
};

// chunks [S][K] u16, glen [G] u32, and for the packed layout each lane's
// bit count and initial state (u16 [K] each)
WsLayout ws_layout(int64_t K, int64_t S) {
    const int64_t G = (K + kLanes - 1) / kLanes;
    WsLayout l;
    l.chunks = 0;
    l.glen = align256(S * K * 2);
    l.plen = l.glen + align256(G * 4);
    l.pstate = l.plen + align256(K * 2);
    l.total = l.pstate + align256(K * 2);
    return l;
}

// Exponent symbol of step i of lane k: the pair e0 * 16 + e1 of bytes 2i,
// 2i + 1, or the exponent of byte i.  Both bytes of a pair lie in the same
// aligned dword (2i is even and so is the row start, N being even); the
// tensor's last dword, which may end past its `total` bytes, is read bytewise.
template <int SPS>
__device__ __forceinline__ uint32_t symbol_at(const uint8_t* __restrict__ fp8, int64_t byte,
                                              int64_t total) {
    const int64_t a = byte & ~int64_t(3);
    uint32_t w;
    if (a + 4 <= total) {
        w = *reinterpret_cast<const uint32_t*>(fp8 + a);
    } else {
        w = 0;
        for (int64_t j = a; j < total; j++) w |= (uint32_t)fp8[j] << (8 * (j - a));
    }
    const uint32_t sh = (uint32_t)(byte & 3) * 8u;
    if constexpr (SPS == 2) {
        return (((w >> (sh + 3)) & 0xFu) << 4) | ((w >> (sh + 11)) & 0xFu);
    } else {
        return (w >> (sh + 3)) & 0xFu;
    }
}

// Per-symbol step constants (the FSE formulation of the same construction).
// For x in [L, 2L) the step emits the nb low bits of x with x >> nb in
// [f, 2f): nb = (x + dnb) >> 16 with maxb = log2L - floor(log2(f - 1))
// (log2L for f = 1) and dnb = (maxb << 16) - (f << maxb); then x = next[idx]
// with idx = start + (x >> nb) - f = (x >> nb) + dfind.  This gives the same
// nb as floor(log2 x) - floor(log2 f), less one when x >> nb < f, for every
// f in [1, L] and x in [L, 2L).  A symbol of frequency 0 is encoded as if
// f = 1 (every index stays in range) and flagged in bit 31 of dnb.
__device__ __forceinline__ uint2 enc_consts(uint32_t e, int log2L) {
    uint32_t f = e & 0xFFFFu;
    const uint32_t start = e >> 16;
    const uint32_t bad = f == 0 ? 1u : 0u;
    if (f == 0) f = 1;
    const uint32_t maxb = f == 1 ? (uint32_t)log2L
                                 : (uint32_t)log2L - (31u - (uint32_t)__builtin_clz(f - 1u));
    const uint32_t dnb = (maxb << 16) - (f << maxb);
    return uint2{dnb | (bad << 31), start - f};
}

// One backward encode step of symbol s: emit the chunk of step i (value in
// bits 11:0, nb in bits 15:12), then x = L + the slot of s's rank-th
// occurrence.  bad collects the flags of the symbols seen.
// The chunk goes to row i of chunks [S][K] through a buffer resource on that
// row (a scalar base; the lane's offset k * 2 is fixed), so the store costs
// no per-step address arithmetic.
__device__ __forceinline__ void enc_step(uint32_t s, const uint2* tab, const uint16_t* nx,
                                         uint32_t L, uint32_t& x, uint32_t& bad, uint32_t& bits,
                                         uint16_t* __restrict__ chunks, int64_t i, int64_t K,
                                         uint32_t koff) {
    const uint2 e = tab[s];
    bad |= e.x;
    const uint32_t nb = __builtin_amdgcn_ubfe(x + e.x, 16u, 5u);
    bits += nb;
    const uint32_t ch = __builtin_amdgcn_ubfe(x, 0u, nb) | (nb << 12);
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)ch,
                                          __builtin_amdgcn_make_buffer_rsrc(chunks + i * K, (short)0,
                                                                            (int)(K * 2),
                                                                            0x00020000),
                                          koff, 0, 0);
    uint32_t idx = (x >> nb) + e.y;
    idx = idx < L ? idx : L - 1u;
    x = nx[idx];
}

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef uint64_t Mask;   // a lane mask of the wave
constexpr int kEncBlockChunks = 8;   // 16-byte chunks per 128-byte block of a row

// Symbol of step q of a 16-byte chunk: bytes 2q, 2q + 1 (pair) or byte q.
template <int SPS, int Q>
__device__ __forceinline__ uint32_t chunk_symbol(const v4u& c) {
    const uint32_t w = c[Q * SPS / 4];
    constexpr uint32_t sh = (uint32_t)((Q * SPS) % 4) * 8u;
    if constexpr (SPS == 2) {
        return (((w >> (sh + 3)) & 0xFu) << 4) | ((w >> (sh + 11)) & 0xFu);
    } else {
        return (w >> (sh + 3)) & 0xFu;
    }
}

// The two sign/mantissa words of a 16-byte tile: sign and mantissa bits
// (mask 0x87 of each byte) of bytes 0-3 in place and of bytes 4-7 rotated
// by 4 bits into the exponent positions, the same for bytes 8-15.
__device__ __forceinline__ void sm_words(const uint32_t (&b)[4], uint32_t& w0, uint32_t& w1) {
    const uint32_t m = 0x87878787u;
    w0 = (b[0] & m) | __builtin_amdgcn_alignbit(b[1] & m, b[1] & m, 28u);
    w1 = (b[2] & m) | __builtin_amdgcn_alignbit(b[3] & m, b[3] & m, 28u);
}

// Chunks top - 1, top - 2, ... of a row into b[0], b[1], ... (zero below 0).
__device__ __forceinline__ void load_block(v4u (&b)[kEncBlockChunks], const v4u* rp,
                                           int64_t top) {
    #pragma unroll
    for (int c = 0; c < kEncBlockChunks; c++) {
        const int64_t j = top - 1 - c;
        b[c] = j >= 0 ? rp[j] : v4u{0u, 0u, 0u, 0u};   // wave-uniform condition
    }
}

// The refill schedule (schedule.h): every lane in range starts with two
// words (64 bits); each segment of steps (2 steps, or 3, 3, 2 per 8 with
// 2^11-state tables) consumes its nb bits, and after a segment that is not
// the last, a lane holding at most 32 bits takes the next word (+32 bits);
// after the second-to-last segment only a lane holding fewer bits than the
// last segment can read (final_below) does.  A segment consumes at most 30
// bits, so after every check but the final one a lane holds 33..64 bits:
// with c the bits consumed so far it has taken floor(c / 32) + 2 words.
// The words a lane takes in all are therefore fixed by its bit count up to
// the third-to-last segment (c3) and up to the second-to-last (c2):
// t = floor(c3 / 32) + 2, plus one when 32 t - c2 < final_below (t = 2,
// c3 = 0 with two segments; 2 words with one segment; none for S = 0).  The
// walk records its bit count after the last segment (b1: bits of the last
// segment's steps) and after the second-to-last (b2: the last two
// segments'), so c2 = bits - b1 and c3 = bits - b2.
__device__ __forceinline__ uint32_t lane_words(int64_t S, bool triple, uint32_t bits,
                                               uint32_t b1, uint32_t b2) {
    if (S == 0) return 0u;
    const int64_t n = tans_sched::segments(S, triple);
    if (n == 1) return 2u;
    const uint32_t c2 = bits - b1;
    const uint32_t c3 = n >= 3 ? bits - b2 : 0u;
    const uint32_t t = c3 / 32u + 2u;
    return t + (32u * t - c2 < (uint32_t)tans_sched::final_below(S, triple) ? 1u : 0u);
}

// One thread per lane walks its row backwards.  When rows are 16-byte
// aligned (N % 16 == 0) a lane loads its row 128 bytes at a time and the
// next 128 bytes while it encodes the current ones: a step then waits on
// LDS only, not on a global load, and each line of the row is fetched in
// one go (the lanes' rows are N bytes apart, so a line read piecewise over
// many steps could leave the cache in between).  A wave is one 64-lane
// group (blocks hold four); its lanes' word counts are summed into
// glen[group], padded to a multiple of 4.  PACKED (the packed layout):
// plen[k] gets the lane's bits (12 for the state + its steps' nb), and
// glen[group] the words of the group's stream (header, bits, padding to 16
// bytes); `states` is then the workspace's state array.
template <int SPS, bool PACKED = false>
__global__ __launch_bounds__(kEncBlock) void enc_backward_kernel(
    const uint8_t* __restrict__ fp8, int64_t K, int64_t N, const uint32_t* __restrict__ enc_tab,
    const uint16_t* __restrict__ next, int log2L, uint16_t* __restrict__ chunks,
    uint16_t* __restrict__ states, uint32_t* __restrict__ glen, uint32_t* __restrict__ sm,
    int* __restrict__ status, uint16_t* __restrict__ plen) {
    static_assert(kEncBlock % kLanes == 0, "blocks hold whole groups");
    constexpr int NSYM = SPS == 2 ? 256 : 16;
    __shared__ uint2 tab[NSYM];
    __shared__ uint16_t nx[1 << TANS_PAIR_LOG2L];
    const uint32_t L = 1u << log2L;
    for (int i = threadIdx.x; i < NSYM; i += blockDim.x) tab[i] = enc_consts(enc_tab[i], log2L);
    for (uint32_t i = threadIdx.x; i < L; i += blockDim.x) nx[i] = next[i];
    __syncthreads();
    const int64_t k = (int64_t)blockIdx.x * kEncBlock + threadIdx.x;
    if (k - (threadIdx.x & (kLanes - 1)) >= K) return;   // the whole group is out of range
    const int64_t S = N / SPS;
    constexpr bool kTriple = SPS == 1;   // 2^11-state tables: 3-3-2 segments
    uint32_t words = 0;
    if (k < K) {
        const int64_t row = k * N;
        uint32_t x = L;
        uint32_t bad = 0;    // bit 31: a symbol of frequency 0
        uint32_t bits = 0;          // the lane's stream bits
        uint32_t b1 = 0, b2 = 0;    // bits of the last segment, of the last two (lane_words)
        const uint32_t koff = (uint32_t)k * 2u;   // K <= INT32_MAX (checked by the launcher)
        if (N % 16 == 0) {   // kernel-uniform
            // S is a multiple of 8 (pair) or 16 (nibble), so the last two
            // segments (steps S - 4 .. or S - 5 ..) are the walk's first
            // steps, all in the row's last chunk
            constexpr int kQ = 16 / SPS;   // steps per chunk
            constexpr int kB2 = kTriple ? kQ - 5 : kQ - 4;   // first step of the last two
            const v4u* rp = reinterpret_cast<const v4u*>(fp8 + row);
            const int64_t nch = N / 16;
            v4u cur[kEncBlockChunks], nxt[kEncBlockChunks];
            load_block(cur, rp, nch);
            for (int64_t hi = nch; hi > 0; hi -= kEncBlockChunks) {
                load_block(nxt, rp, hi - kEncBlockChunks);
                #pragma unroll
                for (int c = 0; c < kEncBlockChunks; c++) {
                    const int64_t j = hi - 1 - c;
                    if (j < 0) break;   // wave-uniform
                    static_for<0, kQ>([&](auto Q) {
                        constexpr int q = kQ - 1 - decltype(Q)::value;
                        enc_step(chunk_symbol<SPS, q>(cur[c]), tab, nx, L, x, bad, bits, chunks,
                                 j * kQ + q, K, koff);
                        if constexpr (q == kQ - 2) {
                            if (j == nch - 1) b1 = bits;   // wave-uniform
                        } else if constexpr (q == kB2) {
                            if (j == nch - 1) b2 = bits;
                        }
                    });
                    // the chunk is tile j: its sign/mantissa words (a wave's
                    // stores cover 512 contiguous bytes)
                    const uint32_t tb[4] = {cur[c].x, cur[c].y, cur[c].z, cur[c].w};
                    uint32_t w0, w1;
                    sm_words(tb, w0, w1);
                    *reinterpret_cast<uint2*>(sm + (j * K + k) * 2) = uint2{w0, w1};
                }
                #pragma unroll
                for (int c = 0; c < kEncBlockChunks; c++) cur[c] = nxt[c];
            }
        } else {
            // first steps of the last segment and of the one before it
            const int64_t n_seg = tans_sched::segments(S, kTriple);
            const int64_t last = tans_sched::seg_start(n_seg - 1, kTriple);
            const int64_t last2 = n_seg >= 2 ? tans_sched::seg_start(n_seg - 2, kTriple) : -1;
            for (int64_t i = S - 1; i >= 0; i--) {
                enc_step(symbol_at<SPS>(fp8, row + i * SPS, K * N), tab, nx, L, x, bad, bits,
                         chunks, i, K, koff);
                if (i == last) b1 = bits;
                if (i == last2) b2 = bits;
            }
        }
        states[k] = (uint16_t)x;
        if (bad >> 31) *status = TANS_ESYMBOL;   // vector store: any failing lane may write it
        if constexpr (PACKED) {
            words = (uint32_t)tans_pack::kStateBits + bits;   // the lane's bits
            plen[k] = (uint16_t)words;
        } else {
            words = lane_words(S, kTriple, bits, b1, b2);
        }
    }
    #pragma unroll
    for (int m = 32; m >= 1; m >>= 1) words += __shfl_xor(words, m, kLanes);
    if ((threadIdx.x & (kLanes - 1)) == 0) {
        if constexpr (PACKED)   // header + bits, padded to 16 bytes
            glen[k / kLanes] = ((uint32_t)tans_pack::hdr_total(S) + (words + 7u) / 8u + 15u) / 16u * 4u;
        else
            glen[k / kLanes] = (words + 3u) & ~3u;
    }
}

// offsets[g] = sum of glen[0..g), offsets[G] = total; one workgroup: each
// thread sums a contiguous run, then a Hillis-Steele scan over the threads.
__global__ __launch_bounds__(1024) void enc_scan_kernel(const uint32_t* __restrict__ glen,
                                                        int64_t G, int64_t* __restrict__ offsets) {
    __shared__ int64_t part[1024];
    const int tid = threadIdx.x;
    const int64_t per = (G + 1023) / 1024;
    const int64_t b = tid * per;
    int64_t sum = 0;
    for (int64_t i = b; i < b + per && i < G; i++) sum += glen[i];
    part[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int64_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    if (tid == 1023) offsets[G] = part[1023];
    int64_t run = part[tid] - sum;
    for (int64_t i = b; i < b + per && i < G; i++) {
        offsets[i] = run;
        run += glen[i];
    }
}

// Zero n words (a kernel rather than hipMemsetAsync, so a caller may
// capture the encoder in a graph).
__global__ __launch_bounds__(kEncBlock) void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kEncBlock + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// One wave per group replays the refill schedule while each lane packs its
// chunks into 32-bit words, LSB first.  A word's place in the stream is
// fixed when the lane takes it: the first two words of every lane are the
// first 2 x lanes words (first words in lane order, then the second), and
// a word taken after a segment goes to handed + rank (ballot + mbcnt, the
// order the decoders read it).  A word is stored when its last bit is
// packed, which comes after it is taken (a segment adds at most 30 bits,
// and a lane takes a word only once it holds at most 32), so each lane
// keeps the places of at most two taken, unfinished words.  Words taken
// past the lane's bits, and the group's padding to 4 words, are zero.  The
// stores go through a buffer resource bounded by the group's length.
// TRIPLE: 2^11-state tables, segments of 3, 3, 2 steps (schedule.h).
constexpr int kPlaceSteps = 16;   // steps whose chunks are loaded together (whole segments)

template <bool TRIPLE>
__global__ __launch_bounds__(kEncBlock) void enc_place_kernel(
    const uint16_t* __restrict__ chunks, int64_t K, int64_t S,
    const int64_t* __restrict__ offsets, uint32_t* __restrict__ comp) {
    // segments per kPlaceSteps steps, and their first steps and lengths
    constexpr int kSegs = TRIPLE ? 6 : 8;
    constexpr auto seg_first = [](int q) { return TRIPLE ? 8 * (q / 3) + 3 * (q % 3) : 2 * q; };
    constexpr auto seg_len = [](int q) { return TRIPLE ? (q % 3 == 2 ? 2 : 3) : 2; };
    static_assert(seg_first(kSegs - 1) + seg_len(kSegs - 1) == kPlaceSteps, "whole segments");
    const int lane = threadIdx.x & (kLanes - 1);
    // the group (wave-uniform, so the output resource stays in SGPRs)
    const int64_t g = (int64_t)blockIdx.x * (kEncBlock / kLanes) +
                      __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t G = (K + kLanes - 1) / kLanes;
    if (g >= G) return;
    const int64_t k = g * kLanes + lane;
    const bool active = k < K;
    const int64_t kk = active ? k : K - 1;
    const uint32_t lanes = (uint32_t)(K - g * kLanes < kLanes ? K - g * kLanes : kLanes);
    const int64_t base = offsets[g];
    const int64_t glen = offsets[g + 1] - base;
    const Rsrc out = __builtin_amdgcn_make_buffer_rsrc(
        comp + base, (short)0, (int)(glen > 0x1FFFFFFF ? 0x7FFFFFFF : glen * 4), 0x00020000);
    // S <= 2^24 (checked by the launcher)
    const int n_seg = (int)tans_sched::segments(S, TRIPLE);
    const int32_t fin_below = S > 0 ? tans_sched::final_below(S, TRIPLE) : 0;
    uint64_t acc = 0;   // packed bits not yet stored
    uint32_t n = 0;     // how many
    uint32_t f0 = (uint32_t)lane, f1 = lanes + (uint32_t)lane;   // places of unfinished words
    uint32_t fc = S > 0 && active ? 2u : 0u;                      // how many
    int32_t held = 64;  // bits the lane holds
    uint32_t handed = S > 0 ? 2u * lanes : 0u;
    // the chunks of steps t0 .. t0 + kPlaceSteps - 1 (zero past step S; the
    // loads stay in bounds and unconditional, so a batch's loads leave
    // together), one batch ahead of the packing
    const uint32_t koff = (uint32_t)kk * 2u;   // K <= INT32_MAX (checked by the launcher)
    const int steps = (int)S;
    auto load = [&](uint32_t (&c)[kPlaceSteps], int t0) {
        #pragma unroll
        for (int u = 0; u < kPlaceSteps; u++) {
            const int t = t0 + u;
            const char* row =
                reinterpret_cast<const char*>(chunks + (int64_t)(t < steps ? t : steps - 1) * K);
            const uint32_t v = *reinterpret_cast<const uint16_t*>(row + koff);
            c[u] = t < steps ? v : 0u;   // wave-uniform
        }
    };
    uint32_t c[kPlaceSteps], cn[kPlaceSteps];
    if (steps > 0) load(c, 0);
    for (int t0 = 0; t0 < steps; t0 += kPlaceSteps) {
        if (t0 + kPlaceSteps < steps) load(cn, t0 + kPlaceSteps);   // wave-uniform
        const int j0 = t0 / kPlaceSteps * kSegs;
        #pragma unroll
        for (int q = 0; q < kSegs; q++) {
            const int j = j0 + q;
            if (j >= n_seg) break;   // wave-uniform
            #pragma unroll
            for (int u = seg_first(q); u < seg_first(q) + seg_len(q); u++) {
                const uint32_t nb = c[u] >> 12;
                acc |= (uint64_t)(c[u] & 0xFFFu) << n;
                n += nb;
                held -= (int32_t)nb;
            }
            if (n >= 32) {   // at most one word per segment (n < 32 + 30)
                if (active)
                    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)acc, out, f0 * 4u, 0, 0);
                f0 = f1;
                fc--;
                acc >>= 32;
                n -= 32;
            }
            if (j + 1 < n_seg) {   // wave-uniform: no check after the last segment
                const int32_t below = j + 2 == n_seg ? fin_below : tans_sched::kAtMost + 1;
                const bool need = active && held < below;
                const Mask m = __ballot(need);
                const uint32_t rank = __builtin_amdgcn_mbcnt_hi(
                    (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                if (need) {
                    if (fc == 0) f0 = handed + rank; else f1 = handed + rank;
                    fc++;
                    held += 32;
                }
                handed += (uint32_t)__popcll(m);
            }
        }
        #pragma unroll
        for (int u = 0; u < kPlaceSteps; u++) c[u] = cn[u];
    }
    if (active) {
        if (n > 0) {   // the last, partial word
            __builtin_amdgcn_raw_buffer_store_b32((uint32_t)acc, out, f0 * 4u, 0, 0);
            f0 = f1;
            fc--;
        }
        if (fc >= 1) __builtin_amdgcn_raw_buffer_store_b32(0u, out, f0 * 4u, 0, 0);
        if (fc >= 2) __builtin_amdgcn_raw_buffer_store_b32(0u, out, f1 * 4u, 0, 0);
    }
    // padding up to the 4-word boundary
    if ((int64_t)handed + lane < glen)
        __builtin_amdgcn_raw_buffer_store_b32(0u, out, (handed + (uint32_t)lane) * 4u, 0, 0);
}

// The packed layout: one wave per group.  Each lane reads its bit count
// (plen), the pair's count is the two lanes' sum, and a scan of the counts
// over the wave gives each pair's end; the wave then ORs the header and
// every lane's bits (state minus L, then each step's chunk; even lanes
// forwards from the pair's start, odd lanes bit-reversed backwards from its
// end) into its LDS buffer, which holds the longest possible stream, and
// copies the group's stream words out (zeros past the bits).
constexpr int kPackWords = (int)(tans_pack::max_stream_bytes(tans_pack::kMaxSteps) / 4);

__global__ __launch_bounds__(kEncBlock) void enc_place_packed_kernel(
    const uint16_t* __restrict__ chunks, const uint16_t* __restrict__ pstate,
    const uint16_t* __restrict__ plen, int64_t K, int64_t S, uint32_t L,
    const int64_t* __restrict__ offsets, uint32_t* __restrict__ comp) {
    __shared__ uint32_t bufs[kEncBlock / kLanes][kPackWords];
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = threadIdx.x / kLanes;
    const int64_t g = (int64_t)blockIdx.x * (kEncBlock / kLanes) + wave;
    const int64_t G = (K + kLanes - 1) / kLanes;
    if (g >= G) return;
    uint32_t* b = bufs[wave];
    for (int i = lane; i < kPackWords; i += kLanes) b[i] = 0u;
    const int64_t k = g * kLanes + lane;
    const bool active = k < K;
    const uint32_t len = active ? plen[k] : 0u;
    const uint32_t cnt = len + (uint32_t)__shfl_xor((int)len, 1, kLanes);   // the pair's bits
    uint32_t v = (lane & 1) ? 0u : cnt;
    #pragma unroll
    for (int d = 1; d < kLanes; d <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)v, d, kLanes);
        if (lane >= d) v += y;
    }
    const int hb = tans_pack::hdr_bytes(S);
    const uint32_t end = (uint32_t)tans_pack::hdr_total(S) * 8u + v;
    const uint32_t start = end - cnt;
    // (the wave's LDS accesses execute in order: the zeroing above lands first)
    if (!(lane & 1)) {
        const uint32_t at = (uint32_t)(lane >> 1) * (uint32_t)hb;
        atomicOr(&b[at >> 2], cnt << (8u * (at & 3u)));
    }
    if (active) {
        const bool odd = lane & 1;
        uint32_t o = 0;   // bits of the lane placed so far
        auto put = [&](uint32_t val, uint32_t nb) {
            if (nb == 0) return;
            // odd lanes: the field's bits run backwards, so it sits reversed
            // at [end - o - nb, end - o)
            const uint32_t p = odd ? end - o - nb : start + o;
            const uint32_t f = odd ? __builtin_bitreverse32(val) >> (32u - nb) : val;
            const uint32_t sh = p & 31u;
            atomicOr(&b[p >> 5], f << sh);
            if (sh + nb > 32u) atomicOr(&b[(p >> 5) + 1], f >> (32u - sh));
            o += nb;
        };
        put((uint32_t)pstate[k] - L, (uint32_t)tans_pack::kStateBits);
        for (int64_t s = 0; s < S; s++) {
            const uint32_t c = chunks[s * K + k];
            put(c & 0xFFFu, c >> 12);
        }
    }
    const int64_t base = offsets[g];
    const int64_t glen = offsets[g + 1] - base;
    for (int64_t i = lane; i < glen && i < kPackWords; i += kLanes) comp[base + i] = b[i];
}

// Sign/mantissa tiles: sm[(t K + k) * 8] from bytes [16t, 16t + 16) of row
// k (zero past N).  A workgroup of 4 waves takes 32 rows x 64 tiles: each
// wave reads 8 rows, one row segment of 1 KiB per instruction (lane = tile),
// turns each 16 bytes into the tile's two sm words, and stages them in LDS
// by [tile][row]; after a barrier each wave writes 16 tiles as contiguous
// 256-byte runs of 32 rows.
constexpr int kSmRows = 32;                      // rows per workgroup
constexpr int kSmCols = kLanes;                  // tiles per workgroup
constexpr int kSmPad = kSmRows + 1;              // LDS row stride (records): 2-way banks at most

__global__ __launch_bounds__(kEncBlock) void enc_sm_kernel(const uint8_t* __restrict__ fp8,
                                                           int64_t K, int64_t N, int64_t n_tiles,
                                                           uint32_t* __restrict__ sm) {
    static_assert(kEncBlock == 4 * kLanes && kSmRows % 4 == 0, "4 waves, 8 rows each");
    __shared__ uint2 st[kSmCols * kSmPad];
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = threadIdx.x / kLanes;
    const int64_t col_blocks = (n_tiles + kSmCols - 1) / kSmCols;
    const int64_t rb = blockIdx.x / col_blocks, cb = blockIdx.x % col_blocks;
    const int64_t k0 = rb * kSmRows, t0 = cb * kSmCols;
    const int64_t t = t0 + lane;   // this lane's tile in the load phase
    constexpr int kPerWave = kSmRows / 4;
    #pragma unroll
    for (int u = 0; u < kPerWave; u++) {
        const int r = wave * kPerWave + u;
        const int64_t k = k0 + r;
        uint32_t b[4] = {0u, 0u, 0u, 0u};
        if (k < K && t < n_tiles) {
            const uint8_t* row = fp8 + k * N;
            if (N % kTile == 0) {   // whole, 16-byte aligned tiles
                const uint4 v = *reinterpret_cast<const uint4*>(row + t * kTile);
                b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
            } else {
                #pragma unroll
                for (int q = 0; q < 4; q++) {
                    #pragma unroll
                    for (int y = 0; y < 4; y++) {
                        const int64_t c = t * kTile + 4 * q + y;
                        if (c < N) b[q] |= (uint32_t)row[c] << (8 * y);
                    }
                }
            }
        }
        uint32_t w0, w1;
        sm_words(b, w0, w1);
        st[lane * kSmPad + r] = uint2{w0, w1};
    }
    __syncthreads();
    // store phase: each instruction writes two tiles x 32 rows (lane / 32, lane % 32)
    const int r = lane % kSmRows;
    const int64_t k = k0 + r;
    #pragma unroll
    for (int v = 0; v < kSmCols / 8; v++) {
        const int tt = (wave * (kSmCols / 8) + v) * 2 + lane / kSmRows;
        const int64_t tg = t0 + tt;
        if (k < K && tg < n_tiles)
            *reinterpret_cast<uint2*>(sm + (tg * K + k) * 2) = st[tt * kSmPad + r];
    }
}

}  // namespace

extern "C" {

int tans_gpu_encode_workspace(int64_t K, int64_t N, int32_t log2L, int64_t* workspace_bytes) {
    if (!workspace_bytes || K < 0 || N < 0 || N % 2)
        return fail(TANS_EINVAL, "gpu_encode: need K >= 0 and even N >= 0");
    if (log2L != TANS_PAIR_LOG2L && log2L != TANS_NIBBLE_LOG2L)
        return fail(TANS_EINVAL, "gpu_encode: log2L must be 12 (pair) or 11 (nibble)");
    const int64_t S = log2L == TANS_PAIR_LOG2L ? N / 2 : N;
    *workspace_bytes = ws_layout(K, S).total;
    return TANS_OK;
}

}  // extern "C"

namespace {

// begin of both layouts; packed: states == NULL (the workspace keeps them)
int gpu_encode_begin(const void* fp8, int64_t K, int64_t N, const uint32_t* enc_tab,
                     const uint16_t* enc_next, int32_t log2L, void* workspace,
                     int64_t workspace_bytes, int64_t* offsets, uint16_t* states, void* sm,
                     int32_t* status, void* stream, bool packed) {
    int64_t need = 0;
    int rc = tans_gpu_encode_workspace(K, N, log2L, &need);
    if (rc) return rc;
    if (packed && (log2L != TANS_PAIR_LOG2L || N > 2 * tans_pack::kMaxSteps))
        return fail(TANS_EINVAL, "gpu_encode_packed: needs log2L 12 and N <= 64");
    if (K == 0 || N == 0) {
        if (K == 0 && offsets) {   // offsets = {0}
            hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kEncBlock), 0, (hipStream_t)stream,
                               reinterpret_cast<uint32_t*>(offsets), (int64_t)2);
            return hip_check(hipGetLastError(), "gpu_encode offsets");
        }
        return fail(TANS_EINVAL, "gpu_encode: N must be positive when K > 0");
    }
    if (!fp8 || !enc_tab || !enc_next || !workspace || !offsets || (!states && !packed) || !sm ||
        !status)
        return fail(TANS_EINVAL, "gpu_encode: null pointer");
    if (workspace_bytes < need) return fail(TANS_EINVAL, "gpu_encode: workspace too small");
    if (reinterpret_cast<uintptr_t>(fp8) % 16)
        return fail(TANS_EINVAL, "gpu_encode: fp8 must be 16-byte aligned");
    const int sps = log2L == TANS_PAIR_LOG2L ? 2 : 1;
    const int64_t S = N / sps;
    const int64_t G = (K + kLanes - 1) / kLanes;
    const int64_t n_tiles = (N + kTile - 1) / kTile;
    // K within int32 (the kernels' lane offsets) and every grid within the
    // 32-bit work-item count of a launch
    const int64_t sm_blocks = (K + kSmRows - 1) / kSmRows * ((n_tiles + kSmCols - 1) / kSmCols);
    if (K > INT32_MAX || S > (int64_t(1) << 24) || sm_blocks > int64_t(UINT32_MAX) / kEncBlock)
        return fail(TANS_EINVAL, "gpu_encode: tensor too large");
    const WsLayout l = ws_layout(K, S);
    char* ws = static_cast<char*>(workspace);
    uint16_t* chunks = reinterpret_cast<uint16_t*>(ws + l.chunks);
    uint32_t* glen = reinterpret_cast<uint32_t*>(ws + l.glen);
    uint16_t* plen = reinterpret_cast<uint16_t*>(ws + l.plen);
    hipStream_t st = (hipStream_t)stream;
    const unsigned lane_blocks = (unsigned)((K + kEncBlock - 1) / kEncBlock);
    if (packed)
        hipLaunchKernelGGL((enc_backward_kernel<2, true>), dim3(lane_blocks), dim3(kEncBlock), 0,
                           st, (const uint8_t*)fp8, K, N, enc_tab, enc_next, (int)log2L, chunks,
                           reinterpret_cast<uint16_t*>(ws + l.pstate), glen, (uint32_t*)sm,
                           status, plen);
    else if (sps == 2)
        hipLaunchKernelGGL(enc_backward_kernel<2>, dim3(lane_blocks), dim3(kEncBlock), 0, st,
                           (const uint8_t*)fp8, K, N, enc_tab, enc_next, (int)log2L, chunks,
                           states, glen, (uint32_t*)sm, status, plen);
    else
        hipLaunchKernelGGL(enc_backward_kernel<1>, dim3(lane_blocks), dim3(kEncBlock), 0, st,
                           (const uint8_t*)fp8, K, N, enc_tab, enc_next, (int)log2L, chunks,
                           states, glen, (uint32_t*)sm, status, plen);
    if ((rc = hip_check(hipGetLastError(), "enc_backward_kernel launch"))) return rc;
    hipLaunchKernelGGL(enc_scan_kernel, dim3(1), dim3(1024), 0, st, glen, G, offsets);
    if ((rc = hip_check(hipGetLastError(), "enc_scan_kernel launch"))) return rc;
    if (N % 16 == 0) return TANS_OK;   // the backward pass wrote the sign/mantissa tiles
    hipLaunchKernelGGL(enc_sm_kernel, dim3((unsigned)sm_blocks), dim3(kEncBlock), 0, st,
                       (const uint8_t*)fp8, K, N, n_tiles, (uint32_t*)sm);
    return hip_check(hipGetLastError(), "enc_sm_kernel launch");
}

int gpu_encode_finish(int64_t K, int64_t N, int32_t log2L, const void* workspace,
                      const int64_t* offsets, void* comp, int64_t comp_bytes, void* stream,
                      bool packed) {
    int64_t need = 0;
    int rc = tans_gpu_encode_workspace(K, N, log2L, &need);
    if (rc) return rc;
    if (packed && (log2L != TANS_PAIR_LOG2L || N > 2 * tans_pack::kMaxSteps))
        return fail(TANS_EINVAL, "gpu_encode_packed: needs log2L 12 and N <= 64");
    if (!workspace || !offsets || !comp) return fail(TANS_EINVAL, "gpu_encode: null pointer");
    if (comp_bytes < kTailWords * 4 || comp_bytes % 4)
        return fail(TANS_EINVAL, "gpu_encode: comp must hold the stream words and the 1 KiB tail");
    hipStream_t st = (hipStream_t)stream;
    const int64_t words_total = comp_bytes / 4 - kTailWords;
    uint32_t* c32 = static_cast<uint32_t*>(comp);
    if (K > 0 && N > 0) {
        const int sps = log2L == TANS_PAIR_LOG2L ? 2 : 1;
        const int64_t S = N / sps;
        const int64_t G = (K + kLanes - 1) / kLanes;
        const WsLayout l = ws_layout(K, S);
        const char* ws = static_cast<const char*>(workspace);
        const dim3 grid((unsigned)((G + kEncBlock / kLanes - 1) / (kEncBlock / kLanes)));
        const uint16_t* ch = reinterpret_cast<const uint16_t*>(ws + l.chunks);
        if (packed)
            hipLaunchKernelGGL(enc_place_packed_kernel, grid, dim3(kEncBlock), 0, st, ch,
                               reinterpret_cast<const uint16_t*>(ws + l.pstate),
                               reinterpret_cast<const uint16_t*>(ws + l.plen), K, S,
                               (uint32_t)(1u << log2L), offsets, c32);
        else if (sps == 1)   // 2^11-state tables: the 3-3-2 schedule
            hipLaunchKernelGGL(enc_place_kernel<true>, grid, dim3(kEncBlock), 0, st, ch, K, S,
                               offsets, c32);
        else
            hipLaunchKernelGGL(enc_place_kernel<false>, grid, dim3(kEncBlock), 0, st, ch, K, S,
                               offsets, c32);
        if ((rc = hip_check(hipGetLastError(), "enc_place_kernel launch"))) return rc;
    }
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((kTailWords + kEncBlock - 1) / kEncBlock)),
                       dim3(kEncBlock), 0, st, c32 + words_total, kTailWords);
    return hip_check(hipGetLastError(), "gpu_encode tail");
}

}  // namespace

extern "C" {

int tans_gpu_encode_begin(const void* fp8, int64_t K, int64_t N, const uint32_t* enc_tab,
                          const uint16_t* enc_next, int32_t log2L, void* workspace,
                          int64_t workspace_bytes, int64_t* offsets, uint16_t* states, void* sm,
                          int32_t* status, void* stream) {
    return gpu_encode_begin(fp8, K, N, enc_tab, enc_next, log2L, workspace, workspace_bytes,
                            offsets, states, sm, status, stream, false);
}

int tans_gpu_encode_finish(int64_t K, int64_t N, int32_t log2L, const void* workspace,
                           const int64_t* offsets, void* comp, int64_t comp_bytes, void* stream) {
    return gpu_encode_finish(K, N, log2L, workspace, offsets, comp, comp_bytes, stream, false);
}

int tans_gpu_encode_packed_begin(const void* fp8, int64_t K, int64_t N, const uint32_t* enc_tab,
                                 const uint16_t* enc_next, int32_t log2L, void* workspace,
                                 int64_t workspace_bytes, int64_t* offsets, void* sm,
                                 int32_t* status, void* stream) {
    return gpu_encode_begin(fp8, K, N, enc_tab, enc_next, log2L, workspace, workspace_bytes,
                            offsets, nullptr, sm, status, stream, true);
}

int tans_gpu_encode_packed_finish(int64_t K, int64_t N, int32_t log2L, const void* workspace,
                                  const int64_t* offsets, void* comp, int64_t comp_bytes,
                                  void* stream) {
    return gpu_encode_finish(K, N, log2L, workspace, offsets, comp, comp_bytes, stream, true);
}

}  // extern "C"
