// gfx950 kernels of the tANS FP8 library and their C-ABI launchers.
//
// Kernels (the data format is described in include/tans_amd.h):
//   fp8_copy_kernel        16-byte streaming copy, the HBM ceiling
//                          (role of csrc/fp8_memcpy.cu:30-41)
//   fp8_add_kernel         uncompressed FP8 add (csrc/vecadd.cu:41-73)
//   table_kernel           decode table from device spread/freqs
//                          (csrc/tans_decode.cu:23-59 without the host trip)
//   fused_add_kernel<SPS>  decode two encodings + FP8 add
//                          (csrc/vecadd.cu:156-243)
//   decode_kernel<SPS>     decode to FP8 bytes [N, K]
//                          (csrc/tans_decode.cu:125-155)
//
// Decoder design.  One wave64 decodes one 64-lane group; each lane owns one
// tANS state.  The table lives in LDS as 8-byte entries indexed by a byte
// offset kept in the state register, so one step is: ds_read_b64, bit-field
// extract of nb bits from a 64-bit LSB-first bit buffer, a 64-bit shift, and
// one shift-add for the next table offset.  Every second step the lane
// refills 32 bits from its next word row when 32 or fewer bits remain (two
// steps read at most 2*12 bits).  The next word is always loaded one refill
// ahead.  FP8 bytes are rebuilt four at a time: the table carries each
// exponent pre-shifted to bits 6:3 of a byte, a v_perm gathers four of them,
// and one v_bfi merges the sign/mantissa word.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/tans_amd.h"

extern "C" void tans_internal_set_error(const char* msg);  // codec.cpp

namespace {

constexpr int kLanes = 64;
constexpr int kTile = 16;
constexpr int kBlock = 256;                 // 4 waves = 4 groups per workgroup
constexpr uint32_t kExpMask = 0x78787878u;  // exponent field of 4 FP8 bytes

// ---------------------------------------------------------------------
// FP8 E4M3FN add of 4 packed bytes.  The bytes go to f16 pairs (exact), are
// added with v_pk_add_f16 (the f16 sum of two E4M3 values rounds only where
// the E4M3 rounding cannot be affected: the dropped bits lie below a quarter
// of an E4M3 ulp), clamped to +-448 with IEEE-754-2019 maximum/minimum so a
// NaN stays NaN, and converted back with round-to-nearest-even.  The gfx950
// conversions do not saturate (an out-of-range value becomes NaN), hence the
// clamp.  Shared by the raw and fused kernels so both give the same bytes.
// ---------------------------------------------------------------------
typedef float v2f __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v2h sat448(v2h v) {
    const v2h lo = {(_Float16)-448.0f, (_Float16)-448.0f};
    const v2h hi = {(_Float16)448.0f, (_Float16)448.0f};
    return __builtin_elementwise_minimum(__builtin_elementwise_maximum(v, lo), hi);
}

__device__ __forceinline__ uint32_t add4_fp8(uint32_t a, uint32_t b) {
    const v2h a01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(a, 1.0f, false);
    const v2h a23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(a, 1.0f, true);
    const v2h b01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b, 1.0f, false);
    const v2h b23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b, 1.0f, true);
    v2s r = {0, 0};
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r, sat448(a01 + b01), 1.0f, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r, sat448(a23 + b23), 1.0f, true);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ v4u add16_fp8(v4u a, v4u b) {
    v4u r;
    r.x = add4_fp8(a.x, b.x);
    r.y = add4_fp8(a.y, b.y);
    r.z = add4_fp8(a.z, b.z);
    r.w = add4_fp8(a.w, b.w);
    return r;
}

// ---------------------------------------------------------------------
// Streaming kernels: each thread moves kUnroll 16-byte vectors, strided by
// the block so every load instruction of a wave covers 1 KiB.
// ---------------------------------------------------------------------
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kBlock) void fp8_copy_kernel(const v4u* __restrict__ a,
                                                          v4u* __restrict__ c, int64_t n_vec) {
    const int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x;
    v4u v[kUnroll];
    #pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const int64_t i = base + (int64_t)u * kBlock;
        if (i < n_vec) v[u] = __builtin_nontemporal_load(a + i);
    }
    #pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const int64_t i = base + (int64_t)u * kBlock;
        if (i < n_vec) __builtin_nontemporal_store(v[u], c + i);
    }
}

__global__ __launch_bounds__(kBlock) void fp8_add_kernel(const v4u* __restrict__ a,
                                                         const v4u* __restrict__ b,
                                                         v4u* __restrict__ c, int64_t n_vec) {
    const int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x;
    v4u va[kUnroll], vb[kUnroll];
    #pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const int64_t i = base + (int64_t)u * kBlock;
        if (i < n_vec) {
            va[u] = __builtin_nontemporal_load(a + i);
            vb[u] = __builtin_nontemporal_load(b + i);
        }
    }
    #pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const int64_t i = base + (int64_t)u * kBlock;
        if (i < n_vec) __builtin_nontemporal_store(add16_fp8(va[u], vb[u]), c + i);
    }
}

// ---------------------------------------------------------------------
// Decode table on the device.  One workgroup; thread s owns symbol s and
// walks the spread in slot order to number its occurrences.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void table_kernel(const int32_t* __restrict__ spread,
                                                    const int32_t* __restrict__ freqs, int nsym,
                                                    int log2L, uint2* __restrict__ table) {
    __shared__ int32_t sp[1 << TANS_PAIR_LOG2L];
    const uint32_t L = 1u << log2L;
    for (uint32_t i = threadIdx.x; i < L; i += blockDim.x) sp[i] = spread[i];
    __syncthreads();
    const int s = threadIdx.x;
    if (s >= nsym) return;
    const uint32_t f = (uint32_t)freqs[s];
    const uint32_t ex = (nsym == 256) ? ((((uint32_t)s >> 4) << 11) | (((uint32_t)s & 0xFu) << 19))
                                      : ((uint32_t)s << 11);
    uint32_t rank = 0;
    for (uint32_t slot = 0; slot < L; slot++) {
        if (sp[slot] != s) continue;
        const uint32_t xp = f + rank++;
        const int nb = xp ? log2L - (31 - __builtin_clz(xp)) : 0;
        const uint32_t base = xp << nb;
        table[slot] = make_uint2((uint32_t)nb | ex, (base - L) * 8u);
    }
}

// ---------------------------------------------------------------------
// Per-lane tANS decoder and the wave's staged word stream.
//
// A group's words are consumed strictly in stream order, so the wave stages
// them through a 512-word LDS ring: segment s (stream words 256s..256s+255)
// lives in ring half s&1 and is loaded with one 16-byte load per lane two
// segments ahead of use.  At a refill check the lanes that need bits take
// consecutive words: lane rank from mbcnt over the ballot, the wave position
// advanced by its popcount.
// ---------------------------------------------------------------------
constexpr int kRefillBelow = 24;   // refill a lane holding fewer bits than this
constexpr int kSegWords = 256;     // 64 lanes x 16 bytes
constexpr int kRingWords = 2 * kSegWords;

struct WaveStream {
    const uint32_t* comp;   // whole compressed buffer
    int64_t seg_base;       // word index of segment 0 of this group
    int64_t max_start;      // last legal segment start (buffer words - 256)
    uint32_t* ring;         // this wave's ring (LDS)
    uint32_t pos;           // next unconsumed stream word
    uint32_t boundary;      // pos at which the oldest ring segment is free
    uint32_t next_seg;      // segment index held in `pend`
    v4u pend;               // segment next_seg, in flight
};

__device__ __forceinline__ v4u load_segment(const WaveStream& s, uint32_t seg, int lane) {
    int64_t start = s.seg_base + (int64_t)seg * kSegWords;
    start = start < 0 ? 0 : (start > s.max_start ? s.max_start : start);
    return __builtin_nontemporal_load(reinterpret_cast<const v4u*>(s.comp + start) + lane);
}

__device__ __forceinline__ void store_segment(WaveStream& s, uint32_t seg, v4u v, int lane) {
    reinterpret_cast<v4u*>(s.ring + (seg & 1u) * kSegWords)[lane] = v;
}

__device__ __forceinline__ void stream_init(WaveStream& s, const uint32_t* comp, int64_t comp_words,
                                            int64_t start, uint32_t* ring, int lane) {
    s.comp = comp;
    s.seg_base = start;
    s.max_start = comp_words - kSegWords;
    s.ring = ring;
    s.pos = 0;
    s.boundary = kSegWords;
    const v4u s0 = load_segment(s, 0, lane);
    const v4u s1 = load_segment(s, 1, lane);
    store_segment(s, 0, s0, lane);
    store_segment(s, 1, s1, lane);
    s.next_seg = 2;
    s.pend = load_segment(s, 2, lane);
}

struct LaneDec {
    uint64_t buf;   // unread bits, LSB first
    uint32_t cnt;   // bits 7:0 = valid bits in buf (upper bits: junk)
    uint32_t x8;    // (state - L) * 8: byte offset of the table entry
};

// Refill check: lanes with fewer than 24 bits take the next stream words.
__device__ __forceinline__ void refill(LaneDec& d, WaveStream& s, bool active, int lane) {
    const bool need = active && (d.cnt & 0xFFu) < (uint32_t)kRefillBelow;
    const uint64_t m = __ballot(need);
    if (m == 0) return;
    if (need) {
        const uint32_t idx = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, s.pos));
        const uint32_t w = s.ring[idx & (kRingWords - 1)];
        d.buf |= (uint64_t)w << (d.cnt & 63u);
        d.cnt += 32u;
    }
    s.pos += (uint32_t)__popcll(m);
    if (s.pos >= s.boundary) {
        // the oldest segment is consumed: its half takes the pending one
        store_segment(s, s.next_seg, s.pend, lane);
        s.next_seg += 1;
        s.pend = load_segment(s, s.next_seg, lane);
        s.boundary += kSegWords;
    }
}

// One tANS step.  Returns the table's word0 (nb and the exponent bytes).
__device__ __forceinline__ uint32_t dec_step(LaneDec& d, const uint2* __restrict__ tbl) {
    const uint2 e = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(tbl) + d.x8);
    const uint32_t bits = __builtin_amdgcn_ubfe((uint32_t)d.buf, 0u, e.x);  // width = e.x[4:0]
    d.buf >>= (e.x & 63u);
    d.x8 = (bits << 3) + e.y;
    d.cnt -= e.x;   // bits 7:0 drop by nb; exponent bytes only touch bits 8+
    return e.x;
}

// Exponent fields of four consecutive elements, from two pair steps or four
// nibble steps (byte 1 of word0 holds the first exponent, byte 2 the second).
__device__ __forceinline__ uint32_t exp4_pair(uint32_t e0, uint32_t e1) {
    return __builtin_amdgcn_perm(e1, e0, 0x06050201u);
}
__device__ __forceinline__ uint32_t exp4_nib(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3) {
    const uint32_t lo = __builtin_amdgcn_perm(e1, e0, 0x0c0c0501u);
    const uint32_t hi = __builtin_amdgcn_perm(e3, e2, 0x05010c0cu);
    return lo | hi;
}

__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
    return (a & mask) | (b & ~mask);
}

// FP8 bytes of 8 elements from their exponent words and the sm word.
__device__ __forceinline__ void compose8(uint32_t ex_lo, uint32_t ex_hi, uint32_t smw,
                                         uint32_t& out_lo, uint32_t& out_hi) {
    out_lo = bfi(kExpMask, ex_lo, smw);
    out_hi = bfi(kExpMask, ex_hi, __builtin_amdgcn_alignbit(smw, smw, 4u));
}

// Decode one 16-element tile of two streams, their steps interleaved.
template <int SPS>
__device__ __forceinline__ void dec_tile2(LaneDec& da, WaveStream& sa, LaneDec& db, WaveStream& sb,
                                          const uint2* __restrict__ tbl, bool active, int lane,
                                          uint32_t ea[4], uint32_t eb[4]) {
    if constexpr (SPS == 2) {
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            refill(da, sa, active, lane);
            refill(db, sb, active, lane);
            const uint32_t a0 = dec_step(da, tbl);
            const uint32_t b0 = dec_step(db, tbl);
            const uint32_t a1 = dec_step(da, tbl);
            const uint32_t b1 = dec_step(db, tbl);
            ea[q] = exp4_pair(a0, a1);
            eb[q] = exp4_pair(b0, b1);
        }
    } else {
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t a[4], b[4];
            #pragma unroll
            for (int h = 0; h < 2; h++) {
                refill(da, sa, active, lane);
                refill(db, sb, active, lane);
                a[2 * h] = dec_step(da, tbl);
                b[2 * h] = dec_step(db, tbl);
                a[2 * h + 1] = dec_step(da, tbl);
                b[2 * h + 1] = dec_step(db, tbl);
            }
            ea[q] = exp4_nib(a[0], a[1], a[2], a[3]);
            eb[q] = exp4_nib(b[0], b[1], b[2], b[3]);
        }
    }
}

// Decode `n` elements (n <= 16, n even) of one stream into exponent words.
template <int SPS>
__device__ __forceinline__ void dec_tile1(LaneDec& d, WaveStream& s, const uint2* __restrict__ tbl,
                                          bool active, int lane, int n, uint32_t ex[4]) {
    if (n == kTile) {
        if constexpr (SPS == 2) {
            #pragma unroll
            for (int q = 0; q < 4; q++) {
                refill(d, s, active, lane);
                const uint32_t e0 = dec_step(d, tbl);
                const uint32_t e1 = dec_step(d, tbl);
                ex[q] = exp4_pair(e0, e1);
            }
        } else {
            #pragma unroll
            for (int q = 0; q < 4; q++) {
                refill(d, s, active, lane);
                const uint32_t e0 = dec_step(d, tbl);
                const uint32_t e1 = dec_step(d, tbl);
                refill(d, s, active, lane);
                const uint32_t e2 = dec_step(d, tbl);
                const uint32_t e3 = dec_step(d, tbl);
                ex[q] = exp4_nib(e0, e1, e2, e3);
            }
        }
        return;
    }
    // ragged last tile
    ex[0] = ex[1] = ex[2] = ex[3] = 0;
    const int steps = n / SPS;
    for (int q = 0; q < steps; q++) {
        if ((q & 1) == 0) refill(d, s, active, lane);
        const uint32_t e = dec_step(d, tbl);
        if constexpr (SPS == 2) ex[q >> 1] |= ((e >> 8) & 0xFFFFu) << (16 * (q & 1));
        else ex[q >> 2] |= ((e >> 8) & 0xFFu) << (8 * (q & 3));
    }
}

template <uint32_t L>
__device__ __forceinline__ void load_table(uint2* lds, const uint2* __restrict__ table) {
    for (uint32_t i = threadIdx.x; i < L; i += blockDim.x) lds[i] = table[i];
}

constexpr int kWaves = 8;                  // waves (= groups) per workgroup
constexpr int kDecBlock = kWaves * kLanes;

template <int SPS>
__global__ __launch_bounds__(kDecBlock) void fused_add_kernel(
    const uint32_t* __restrict__ a_comp, int64_t a_words, const int64_t* __restrict__ a_off,
    const uint16_t* __restrict__ a_st, const uint2* __restrict__ a_sm,
    const uint32_t* __restrict__ b_comp, int64_t b_words, const int64_t* __restrict__ b_off,
    const uint16_t* __restrict__ b_st, const uint2* __restrict__ b_sm,
    const uint2* __restrict__ table, int64_t K, int64_t n_tiles, v4u* __restrict__ out) {
    constexpr uint32_t L = SPS == 2 ? (1u << TANS_PAIR_LOG2L) : (1u << TANS_NIBBLE_LOG2L);
    __shared__ uint2 tbl[L];
    __shared__ uint32_t rings[kWaves][2][kRingWords];
    load_table<L>(tbl, table);
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t g = (int64_t)blockIdx.x * kWaves + wave;
    const int64_t k = g * kLanes + lane;
    const bool live = g * kLanes < K;   // wave-uniform
    WaveStream sa, sb;
    if (live) {
        stream_init(sa, a_comp, a_words, a_off[g], rings[wave][0], lane);
        stream_init(sb, b_comp, b_words, b_off[g], rings[wave][1], lane);
    }
    __syncthreads();   // table and first ring segments visible
    if (!live) return;
    const bool active = k < K;
    LaneDec da, db;
    da.buf = db.buf = 0;
    da.cnt = db.cnt = 0;
    da.x8 = ((active ? a_st[k] : L) - L) * 8u;
    db.x8 = ((active ? b_st[k] : L) - L) * 8u;
    uint2 sma = active ? a_sm[k] : make_uint2(0, 0);
    uint2 smb = active ? b_sm[k] : make_uint2(0, 0);
    for (int64_t t = 0; t < n_tiles; t++) {
        uint2 na = make_uint2(0, 0), nb = make_uint2(0, 0);
        if (active && t + 1 < n_tiles) {
            na = a_sm[(t + 1) * K + k];
            nb = b_sm[(t + 1) * K + k];
        }
        uint32_t ea[4], eb[4];
        dec_tile2<SPS>(da, sa, db, sb, tbl, active, lane, ea, eb);
        uint32_t wa[4], wb[4];
        compose8(ea[0], ea[1], sma.x, wa[0], wa[1]);
        compose8(ea[2], ea[3], sma.y, wa[2], wa[3]);
        compose8(eb[0], eb[1], smb.x, wb[0], wb[1]);
        compose8(eb[2], eb[3], smb.y, wb[2], wb[3]);
        const v4u va = {wa[0], wa[1], wa[2], wa[3]};
        const v4u vb = {wb[0], wb[1], wb[2], wb[3]};
        if (active) __builtin_nontemporal_store(add16_fp8(va, vb), out + t * K + k);
        sma = na;
        smb = nb;
    }
}

template <int SPS>
__global__ __launch_bounds__(kDecBlock) void decode_kernel(
    const uint32_t* __restrict__ comp, int64_t words, const int64_t* __restrict__ off,
    const uint16_t* __restrict__ st, const uint2* __restrict__ sm,
    const uint2* __restrict__ table, int64_t K, int64_t N, uint8_t* __restrict__ out) {
    constexpr uint32_t L = SPS == 2 ? (1u << TANS_PAIR_LOG2L) : (1u << TANS_NIBBLE_LOG2L);
    __shared__ uint2 tbl[L];
    __shared__ uint32_t rings[kWaves][kRingWords];
    load_table<L>(tbl, table);
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t g = (int64_t)blockIdx.x * kWaves + wave;
    const int64_t k = g * kLanes + lane;
    const bool live = g * kLanes < K;
    WaveStream s;
    if (live) stream_init(s, comp, words, off[g], rings[wave], lane);
    __syncthreads();
    if (!live) return;
    const bool active = k < K;
    LaneDec d;
    d.buf = 0;
    d.cnt = 0;
    d.x8 = ((active ? st[k] : L) - L) * 8u;
    const int64_t n_tiles = (N + kTile - 1) / kTile;
    for (int64_t t = 0; t < n_tiles; t++) {
        const int64_t e0 = t * kTile;
        const int n = (int)(N - e0 < kTile ? N - e0 : kTile);
        const uint2 smw = active ? sm[t * K + k] : make_uint2(0, 0);
        uint32_t ex[4], w[4];
        dec_tile1<SPS>(d, s, tbl, active, lane, n, ex);
        compose8(ex[0], ex[1], smw.x, w[0], w[1]);
        compose8(ex[2], ex[3], smw.y, w[2], w[3]);
        if (active) {
            #pragma unroll
            for (int i = 0; i < kTile; i++) {
                if (i < n) out[(e0 + i) * K + k] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
            }
        }
    }
}

int fail(int code, const std::string& msg) {
    tans_internal_set_error(msg.c_str());
    return code;
}

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return TANS_OK;
    return fail(TANS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

int sps_for(int32_t log2L) {
    return log2L == TANS_PAIR_LOG2L ? 2 : (log2L == TANS_NIBBLE_LOG2L ? 1 : 0);
}

}  // namespace

extern "C" {

int tans_fp8_memcpy(const void* a, void* c, int64_t n, void* stream) {
    if (n < 0 || n % 16 || ((!a || !c) && n)) return fail(TANS_EINVAL, "memcpy: n must be a multiple of 16");
    if (n == 0) return TANS_OK;
    const int64_t n_vec = n / 16;
    const int64_t blocks = (n_vec + (int64_t)kBlock * kUnroll - 1) / ((int64_t)kBlock * kUnroll);
    hipLaunchKernelGGL(fp8_copy_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)stream,
                       (const v4u*)a, (v4u*)c, n_vec);
    return hip_check(hipGetLastError(), "fp8_copy_kernel launch");
}

int tans_fp8_vecadd_raw(const void* a, const void* b, void* c, int64_t n, void* stream) {
    if (n < 0 || n % 16 || ((!a || !b || !c) && n)) return fail(TANS_EINVAL, "vecadd_raw: n must be a multiple of 16");
    if (n == 0) return TANS_OK;
    const int64_t n_vec = n / 16;
    const int64_t blocks = (n_vec + (int64_t)kBlock * kUnroll - 1) / ((int64_t)kBlock * kUnroll);
    hipLaunchKernelGGL(fp8_add_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)stream,
                       (const v4u*)a, (const v4u*)b, (v4u*)c, n_vec);
    return hip_check(hipGetLastError(), "fp8_add_kernel launch");
}

int tans_build_decode_table_device(const int32_t* spread, const int32_t* freqs, int32_t nsym,
                                   int32_t log2L, uint32_t* table, void* stream) {
    if (!spread || !freqs || !table) return fail(TANS_EINVAL, "table: null pointer");
    if (!((nsym == 256 && log2L == TANS_PAIR_LOG2L) || (nsym == 16 && log2L == TANS_NIBBLE_LOG2L)))
        return fail(TANS_EINVAL, "table: need (nsym 256, log2L 12) or (nsym 16, log2L 11)");
    hipLaunchKernelGGL(table_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, spread, freqs,
                       (int)nsym, (int)log2L, (uint2*)table);
    return hip_check(hipGetLastError(), "table_kernel launch");
}

int tans_fp8_vecadd_fused(const void* a_comp, int64_t a_comp_bytes, const int64_t* a_offsets,
                          const uint16_t* a_states, const void* a_sm, const void* b_comp,
                          int64_t b_comp_bytes, const int64_t* b_offsets, const uint16_t* b_states,
                          const void* b_sm, const uint32_t* table, int32_t log2L, int64_t K,
                          int64_t N, void* out, void* stream) {
    const int sps = sps_for(log2L);
    if (!sps) return fail(TANS_EINVAL, "vecadd_fused: log2L must be 12 (pair) or 11 (nibble)");
    if (K < 0 || N < 0 || N % kTile) return fail(TANS_EINVAL, "vecadd_fused: N must be a multiple of 16");
    if (K == 0 || N == 0) return TANS_OK;
    if (!a_comp || !a_offsets || !a_states || !a_sm || !b_comp || !b_offsets || !b_states || !b_sm ||
        !table || !out)
        return fail(TANS_EINVAL, "vecadd_fused: null pointer");
    if (a_comp_bytes % 16 || b_comp_bytes % 16 || a_comp_bytes < kSegWords * 4 ||
        b_comp_bytes < kSegWords * 4)
        return fail(TANS_EINVAL, "vecadd_fused: compressed buffers must be >= 1 KiB and 16-byte multiples");
    const int64_t groups = (K + kLanes - 1) / kLanes;
    const int64_t blocks = (groups + kWaves - 1) / kWaves;
    const int64_t n_tiles = N / kTile;
#define TANS_LAUNCH_FUSED(S)                                                                      \
    hipLaunchKernelGGL(fused_add_kernel<S>, dim3((unsigned)blocks), dim3(kDecBlock), 0,         \
                       (hipStream_t)stream, (const uint32_t*)a_comp, a_comp_bytes / 4,          \
                       a_offsets, a_states, (const uint2*)a_sm, (const uint32_t*)b_comp,        \
                       b_comp_bytes / 4, b_offsets, b_states, (const uint2*)b_sm,               \
                       (const uint2*)table, K, n_tiles, (v4u*)out)
    if (sps == 2) TANS_LAUNCH_FUSED(2);
    else TANS_LAUNCH_FUSED(1);
#undef TANS_LAUNCH_FUSED
    return hip_check(hipGetLastError(), "fused_add_kernel launch");
}

int tans_decode(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                const uint16_t* states, const void* sm, const uint32_t* table, int32_t log2L,
                int64_t K, int64_t N, void* out, void* stream) {
    const int sps = sps_for(log2L);
    if (!sps) return fail(TANS_EINVAL, "decode: log2L must be 12 (pair) or 11 (nibble)");
    if (K < 0 || N < 0 || N % 2) return fail(TANS_EINVAL, "decode: N must be even");
    if (K == 0 || N == 0) return TANS_OK;
    if (!comp || !offsets || !states || !sm || !table || !out)
        return fail(TANS_EINVAL, "decode: null pointer");
    if (comp_bytes % 16 || comp_bytes < kSegWords * 4)
        return fail(TANS_EINVAL, "decode: compressed buffer must be >= 1 KiB and a 16-byte multiple");
    const int64_t groups = (K + kLanes - 1) / kLanes;
    const int64_t blocks = (groups + kWaves - 1) / kWaves;
#define TANS_LAUNCH_DECODE(S)                                                                     \
    hipLaunchKernelGGL(decode_kernel<S>, dim3((unsigned)blocks), dim3(kDecBlock), 0,            \
                       (hipStream_t)stream, (const uint32_t*)comp, comp_bytes / 4, offsets,     \
                       states, (const uint2*)sm, (const uint2*)table, K, N, (uint8_t*)out)
    if (sps == 2) TANS_LAUNCH_DECODE(2);
    else TANS_LAUNCH_DECODE(1);
#undef TANS_LAUNCH_DECODE
    return hip_check(hipGetLastError(), "decode_kernel launch");
}

}  // extern "C"
