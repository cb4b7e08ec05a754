// gfx950 kernels of the tANS FP8 library and their C-ABI launchers (the GPU
// encoder is in encode.hip).
//
// Kernels (the data format is described in include/tans_amd.h):
//   fp8_copy_kernel          16-byte streaming copy, the HBM ceiling
//                            (role of csrc/fp8_memcpy.cu:30-41)
//   fp8_add_kernel           uncompressed FP8 add (csrc/vecadd.cu:41-73)
//   stream_probe_kernel      read-only / write-only / 2:1 streaming at the
//                            add's launch shape (bandwidth ceilings)
//   table_kernel             decode table from device spread/freqs
//                            (csrc/tans_decode.cu:23-59 without the host trip)
//   fused_add_kernel<SPS,G,FIRST> decode two encodings + FP8 add
//                            (csrc/vecadd.cu:156-243)
//   decode_kernel<SPS,FIRST> decode to FP8 bytes [N, K]
//                            (csrc/tans_decode.cu:125-155)
//   gemm_fused_kernel<SPS>   decode W + skinny GEMM partial sums on the
//                            matrix cores (no counterpart in the
//                            reference), with gemm_finalize_kernel and the
//                            uncompressed baselines gemm_raw_xs_kernel
//                            (rows of up to 8192 columns), and for longer
//                            rows gemm_raw_dot2_kernel (B = 1) and
//                            gemm_raw_kernel (B >= 2)
//
// Decoder design.  One wave64 decodes one 64-lane group; each lane owns one
// tANS state.  The decode table lives in LDS as 8-byte entries addressed by
// a byte offset kept in the state register.  A lane's unread bits sit in a
// 64-bit window (hi:lo) read from bit pos of lo (0 <= pos < 32).  Steps go
// in segments (schedule.h): pairs with the pair alphabet, 3, 3 and 2 steps
// per 8 with the nibble alphabet.  One funnel shift takes the 32 bits from
// pos (a segment reads at most 24 or 30), each step is a ds_read_b64 of the
// entry, a bit-field extract of nb bits and one shift-add for the next
// entry's offset, and pos advances by the segment's nb sum in a register
// that holds pos both in bits 4:0 and in bits 31:27 (the table holds nb in
// both places), so the add's carry out is set exactly when lo is used up.
//
// That carry drives the refill: after each segment but the last, the lanes
// whose lo is used up move hi into lo and take the next word of the group's
// stream (the carry mask, an mbcnt for each lane's rank and one ds_read_b32
// from the wave's LDS ring); after the second-to-last segment a lane takes
// a word only when it holds fewer bits than the last segment can read.
// Each lane starts with two words.  The ring holds kSlots segments of 256 words (one 16-byte load per
// lane) plus a 64-word mirror of its first words, so a wave's 64
// consecutive reads never wrap.  A stage issues at most one segment load
// per stream, through a buffer resource whose base is the stream's first
// word and whose bound is the buffer's end, once the segment's ring slot is
// free.  The loaded segment stays in registers and is written into the
// ring at the next stage whose slot is free, which comes no later than the
// stage in which a lane could first take one of its words.  Slots past a
// stream's end are never written: no lane takes a word there.  A stage is at
// most four refill checks, so at most 256 words are handed out per stage, and
// kSlots = kDelay + 2 slots guarantee that a fetched segment starts more
// than a stage's worth of words ahead of the lanes.  Lanes out of range
// (a tensor's last, partial group) step on a sink table entry that reads
// no bits, so the refill needs no mask of the lanes in range.
//
// FP8 bytes are rebuilt four at a time: the table carries each exponent
// pre-shifted to bits 6:3 of a byte, a v_perm gathers four of them and one
// v_bfi merges the sign/mantissa word.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>
#include <string>
#include <type_traits>

#include "../../include/tans_amd.h"
#include "schedule.h"

extern "C" void tans_internal_set_error(const char* msg);  // codec.cpp

namespace {

constexpr int kLanes = 64;
constexpr int kTile = 16;
constexpr uint32_t kExpMask = 0x78787878u;  // exponent field of 4 FP8 bytes

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// ---------------------------------------------------------------------
// FP8 E4M3FN add of 4 packed bytes.  The bytes go to f16 pairs (exact) and
// are added with v_pk_add_f16.  E4M3 has p = 4 significant bits and f16
// p' = 11 >= 2p + 2, so rounding the exact sum first to f16 and then to E4M3
// (both nearest-even) equals a single rounding of the exact sum.  The sum
// is clamped to +-448 with IEEE-754-2019 maximum/minimum (a NaN stays NaN)
// and converted back with round-to-nearest-even: the gfx950 conversions do
// not saturate (an out-of-range value becomes 0x7E/0x7F), hence the clamp.
// Shared by the raw and fused kernels so both give the same bytes.
// ---------------------------------------------------------------------
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

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
    // the first conversion fills bytes 0-1, the second bytes 2-3; `a` only
    // supplies the don't-care initial contents
    v2s r = __builtin_bit_cast(v2s, a);
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
// Streaming kernels: one 16-byte vector per thread and tensor, non-temporal
// loads and stores.  Measured on MI355X this shape moves more bytes per
// second than grid-stride loops or several vectors per thread.
// ---------------------------------------------------------------------
constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void fp8_copy_kernel(const v4u* __restrict__ a,
                                                          v4u* __restrict__ c, int64_t n_vec) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n_vec) __builtin_nontemporal_store(__builtin_nontemporal_load(a + i), c + i);
}

__global__ __launch_bounds__(kBlock) void fp8_add_kernel(const v4u* __restrict__ a,
                                                         const v4u* __restrict__ b,
                                                         v4u* __restrict__ c, int64_t n_vec) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n_vec) {
        const v4u va = __builtin_nontemporal_load(a + i);
        const v4u vb = __builtin_nontemporal_load(b + i);
        __builtin_nontemporal_store(add16_fp8(va, vb), c + i);
    }
}

// Bandwidth probes: the same launch shape with the arithmetic taken out, to
// measure what this shape can stream.  MODE 0 reads a (a load whose XOR
// matches a fixed key stores its index to sink, which keeps the loads
// live); MODE 1 writes c; MODE 2 writes c = a ^ b (the raw add's 2:1 mix).
template <int MODE, bool NT>
__global__ __launch_bounds__(kBlock) void stream_probe_kernel(const v4u* __restrict__ a,
                                                              const v4u* __restrict__ b,
                                                              v4u* __restrict__ c, int64_t n_vec,
                                                              uint32_t* __restrict__ sink) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n_vec) return;
    if constexpr (MODE == 0) {
        const v4u v = NT ? __builtin_nontemporal_load(a + i) : a[i];
        if ((v.x ^ v.y ^ v.z ^ v.w) == 0x9E3779B9u) sink[0] = (uint32_t)i;
    } else if constexpr (MODE == 1) {
        const uint32_t x = (uint32_t)i;
        const v4u v = {x, x ^ 0x55555555u, x ^ 0xAAAAAAAAu, ~x};
        if (NT) __builtin_nontemporal_store(v, c + i); else c[i] = v;
    } else {
        const v4u v = NT ? __builtin_nontemporal_load(a + i) ^ __builtin_nontemporal_load(b + i)
                         : a[i] ^ b[i];
        if (NT) __builtin_nontemporal_store(v, c + i); else c[i] = v;
    }
}

// ---------------------------------------------------------------------
// Decode table on the device: one workgroup of 16 waves.  The L slots are
// cut into segments of 64 (wave w, round r: segment w * rounds + r, so
// segments follow slot order).  A symbol's rank (its earlier slots, in
// slot order) is its count in earlier segments plus its place among equal
// symbols in its own segment.  The lanes holding a lane's symbol are the
// AND over symbol bits of that bit's ballot (complemented where the lane's
// own bit is 0); mbcnt of that mask is the place, its popcount the count,
// and the last lane holding each symbol writes the count to LDS.  An exclusive prefix over segments (16
// segments per thread, then 4 partial totals per symbol) gives the rest.
//
// The kernel checks what the host builder (codec.cpp) checks: frequencies
// not negative and summing to L, every present symbol of a 2^11-state
// table at a frequency of at least 2, spread symbols inside the alphabet
// and each symbol's slot count equal to its frequency (a rank below it).
// On any failure it sets *status (when given) to TANS_ETABLE; the table it
// writes is then wrong but still in range: a symbol outside the alphabet is
// folded into it, and the decoders' table_store replaces entries that
// would step outside the table or read too many bits.
// ---------------------------------------------------------------------
constexpr int kTableWaves = 16;
constexpr int kTableSegs = kTableWaves * 4;   // 64 segments of 64 slots at L = 4096

__global__ __launch_bounds__(kTableWaves * 64) void table_kernel(
    const int32_t* __restrict__ spread, const int32_t* __restrict__ freqs, int nsym, int log2L,
    v2u* __restrict__ table, int32_t* __restrict__ status) {
    __shared__ uint16_t cnt[kTableSegs][256];   // per segment: counts, then exclusive prefix
    __shared__ uint16_t tot[4][256];            // prefix totals of segment quarters
    __shared__ uint32_t fsum, bad;              // sum of the frequencies; any check failed
    const uint32_t L = 1u << log2L;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rounds = (int)(L / (kTableWaves * 64));   // 4 (pair) or 2 (nibble)
    const int sym_bits = 31 - __builtin_clz((uint32_t)nsym);
    const int nseg = kTableWaves * rounds;
    for (uint32_t i = threadIdx.x; i < kTableSegs * 256 / 2; i += blockDim.x)
        reinterpret_cast<uint32_t*>(&cnt[0][0])[i] = 0u;
    if (threadIdx.x == 0) { fsum = 0u; bad = 0u; }
    __syncthreads();
    uint32_t my_bad = 0u;
    if ((int)threadIdx.x < nsym) {
        const int32_t f = freqs[threadIdx.x];
        const int32_t min_f = log2L == tans_sched::kTripleLog2L ? (int32_t)tans_sched::kTripleMinFreq : 1;
        if (f < 0 || f > (int32_t)L || (f > 0 && f < min_f)) my_bad = 1u;
        else atomicAdd(&fsum, (uint32_t)f);
    }
    uint32_t sym[4] = {0u, 0u, 0u, 0u}, rank[4] = {0u, 0u, 0u, 0u};
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        if (r >= rounds) break;
        const int seg = wave * rounds + r;
        // a symbol outside the alphabet is folded into it (and reported)
        const int32_t raw = spread[seg * 64 + lane];
        if (raw < 0 || raw >= nsym) my_bad = 1u;
        const uint32_t sv = (uint32_t)raw & (uint32_t)(nsym - 1);
        sym[r] = sv;
        // the lanes holding the same symbol: for each symbol bit, the ballot
        // of lanes with that bit set, complemented where this lane's bit is 0
        uint32_t mlo = 0xFFFFFFFFu, mhi = 0xFFFFFFFFu;
        #pragma unroll
        for (int bit = 0; bit < 8; bit++) {
            if (bit >= sym_bits) break;
            const uint64_t B = __ballot((sv >> bit) & 1u);
            const uint32_t mine = (uint32_t)__builtin_amdgcn_sbfe((int)sv, bit, 1);   // 0 or ~0
            mlo &= ~((uint32_t)B ^ mine);
            mhi &= ~((uint32_t)(B >> 32) ^ mine);
        }
        const uint32_t rk = __builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
        const uint32_t tot = (uint32_t)__builtin_popcount(mlo) + (uint32_t)__builtin_popcount(mhi);
        rank[r] = rk;
        if (rk + 1u == tot) cnt[seg][sv] = (uint16_t)tot;
    }
    __syncthreads();
    // exclusive prefix over segments: thread (q, s) scans segments [16q, 16q + 16)
    const int s = threadIdx.x & 255;
    const int q = threadIdx.x >> 8;
    uint32_t run = 0;
    if (s < nsym) {
        uint16_t v[16];
        #pragma unroll
        for (int i = 0; i < 16; i++) v[i] = (16 * q + i < nseg) ? cnt[16 * q + i][s] : (uint16_t)0;
        #pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t c = v[i];
            v[i] = (uint16_t)run;
            run += c;
        }
        tot[q][s] = (uint16_t)run;
        #pragma unroll
        for (int i = 0; i < 16; i++)
            if (16 * q + i < nseg) cnt[16 * q + i][s] = v[i];
    }
    __syncthreads();
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        if (r >= rounds) break;
        const int seg = wave * rounds + r;
        const uint32_t sv = sym[r];
        uint32_t before = 0;
        for (int qq = 0; qq < (seg >> 4); qq++) before += tot[qq][sv];
        const uint32_t f = (uint32_t)freqs[sv];
        const uint32_t rk = before + cnt[seg][sv] + rank[r];   // rank among sv's slots
        if (rk >= f) my_bad = 1u;                              // more slots than its frequency
        const uint32_t xp = f + rk;
        const int top = xp ? 31 - __builtin_clz(xp) : log2L;
        const int nb = top < log2L ? log2L - top : 0;
        const uint32_t base = xp << nb;
        const uint32_t ex = (nsym == 256) ? (((sv >> 4) << 11) | ((sv & 0xFu) << 19)) : (sv << 11);
        table[seg * 64 + lane] = v2u{(uint32_t)nb | ex | ((uint32_t)nb << 27), (base - L) * 8u};
    }
    if (my_bad) bad = 1u;   // benign race: every writer stores 1
    __syncthreads();
    if (threadIdx.x == 0 && status && (bad || fsum != L)) *status = TANS_ETABLE;
}

// ---------------------------------------------------------------------
// Buffer resources.  Loads and stores in the decode loops go through raw
// buffer descriptors: a wave-uniform base, a 32-bit lane offset, and a byte
// bound past which loads return zero and stores are dropped (so idle fetch
// slots, lanes past K and malformed offsets never touch memory outside the
// tensors).  0x00020000 is the gfx9-family descriptor word 3 for raw
// 32-bit-element access.
// ---------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kNT = 2;   // cache policy: non-temporal

__device__ __forceinline__ Rsrc rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRsrcWord3);
}

// ---------------------------------------------------------------------
// Decoder building blocks.
// ---------------------------------------------------------------------
typedef v4u Seg;                           // one segment: 16 bytes per lane
constexpr int kSegWords = 4 * kLanes;
constexpr int kChecksPerStage = 4;         // at most 4 refill checks per stage (8 steps)
constexpr int kDelay = 1;                  // stages from a segment load to its earliest ring write
constexpr int kSlots = kDelay + 2;
constexpr int kRingWords = kSlots * kSegWords;
constexpr int kMirrorWords = kLanes;
constexpr int kRingAlloc = kRingWords + kMirrorWords;
constexpr int kDecWaves = 16;              // waves per workgroup
constexpr int kSmAhead = 4;                // sign/mantissa rows are loaded this many tiles ahead
constexpr int kDecBlock = kDecWaves * kLanes;
// At most kChecksPerStage * 64 words are handed out per stage.  A segment is
// fetched once the one kSlots earlier in its slot is consumed; it can be
// written kDelay stages later at the earliest and is first read no earlier
// than (kSlots - 1) * kSegWords - kChecksPerStage * 64 words after the fetch
// decision.
static_assert((kSlots - 1) * kSegWords >= (kDelay + 1) * kChecksPerStage * kLanes,
              "ring too small for the delay");
// A streaming chain may also start with only its first kLazySegs segments in
// the ring (the GEMM kernel): the next one is fetched at
// the first stage.  The lanes take two words each at the start and at most a
// stage's worth before the second stage, which is where that segment can
// first be written, so they stay inside the segments already there.
constexpr int kLazySegs = 2;
static_assert(kLazySegs < kSlots &&
                  kLazySegs * kSegWords >= 2 * kLanes + kChecksPerStage * kLanes,
              "a lazy start must cover the first stage");

// State of one group's word stream.  Everything but ring_w is wave-uniform.
struct Feed {
    Rsrc src;               // the stream: base at its first word, bound at the buffer's end
    uint32_t next_b;        // byte offset in the stream of the next segment to fetch
    uint32_t len_b;         // bytes in the stream (clamped to the buffer)
    uint32_t next_slot;     // ring slot of the next segment
    uint32_t dest;          // ring slot of the pending segment
    uint32_t pend_new;      // 1 while the pending segment is not in the ring
    uint32_t handed;        // words handed to lanes so far
    uint32_t ring_b;        // byte offset in the ring of word `handed`
    uint32_t ring_w;        // LDS word index of the ring, held in a VGPR (see refill)
    uint32_t* ring;         // this wave's ring for this stream (LDS)
};

// Per-lane decoder state.
struct Lane {
    uint32_t lo, hi;   // 64-bit window of stream bits; the next unread bit is bit pos of lo
    uint32_t q;        // pos (0..31) in bits 4:0 and again in bits 31:27; bits 26:5 scratch
    uint32_t x8;       // (state - L) * 8: byte offset of the state's table entry
};

// A copy of a wave-uniform value in a VGPR (an operand of a VALU
// instruction that already reads an SGPR must be a VGPR).
__device__ __forceinline__ uint32_t in_vgpr(uint32_t x) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(x));
    return v;
}

// Byte offset that reads nothing: every stream bound is below 2^31.
constexpr uint32_t kNoSeg = 0x80000000u;

// The segment at byte offset b of the stream: the lane's 16 bytes, zeros
// past the buffer's end.
__device__ __forceinline__ Seg fetch_seg(const Feed& f, uint32_t b, int lane) {
    return __builtin_amdgcn_raw_buffer_load_b128(f.src, (uint32_t)lane * 16u + b, 0, 0);
}

__device__ __forceinline__ void write_seg(uint32_t* ring, uint32_t slot, Seg v, int lane) {
    reinterpret_cast<Seg*>(ring + slot * kSegWords)[lane] = v;
    if (slot == 0 && lane < kMirrorWords / 4)
        reinterpret_cast<Seg*>(ring + kRingWords)[lane] = v;
}

// Clamp a group's stream (words s .. e of comp) to the buffer and fetch its
// first NSEG segments into `first`: kSlots, kLazySegs (the stage fetches
// continue from segment NSEG), or fewer for streams known to fit them.
// Segments past the stream's end are loads with an empty range,
// which read nothing.  feed_commit writes them to the ring.  The two halves
// let a kernel
// issue these loads together with the decode table's, so the stream and the
// table cost one memory round trip before decoding starts.  Callers read the
// stream offsets of all their chains before the first call, so those scalar
// loads share one round trip too.  lds0 is the start of the workgroup's LDS
// (the decode table).
template <int NSEG = kSlots>
__device__ __forceinline__ void feed_fetch(Feed& f, const uint32_t* comp, int64_t words,
                                           int64_t s, int64_t e, uint32_t* ring,
                                           const void* lds0, int lane, Seg (&first)[kSlots]) {
    s = s < 0 ? 0 : (s > words ? words : s);
    e = e < s ? s : (e > words ? words : e);
    const int64_t room = (words - s) * 4;
    const uint32_t bound = room > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)room;
    const int64_t len = (e - s) * 4;
    f.src = rsrc(comp + s, bound);
    f.len_b = len > (int64_t)bound ? bound : (uint32_t)len;
    f.next_b = (uint32_t)(NSEG * kSegWords * 4);
    f.next_slot = (uint32_t)(NSEG % kSlots);
    f.ring = ring;
    f.ring_w = in_vgpr((uint32_t)(reinterpret_cast<const char*>(ring) -
                                  reinterpret_cast<const char*>(lds0)) / 4u);
    #pragma unroll
    for (int i = 0; i < NSEG; i++) {
        const uint32_t b = (uint32_t)(i * kSegWords * 4);
        first[i] = fetch_seg(f, b < f.len_b ? b : kNoSeg, lane);
    }
}

// Slots past the stream's end stay unwritten (wave-uniform tests).  With
// NSEG = kSlots the last of the first segments becomes the pending one,
// already in the ring (see feed_stage).  With NSEG < kSlots (a lazy start,
// or streams known to fit NSEG segments, decoded without feed_stage) only
// those are loaded and written, and no segment is pending.
template <int NSEG = kSlots>
__device__ __forceinline__ void feed_commit(Feed& f, int lane, const Seg (&first)[kSlots],
                                            Seg& pend) {
    #pragma unroll
    for (int i = 0; i < NSEG; i++)
        if (i == 0 || (uint32_t)(i * kSegWords * 4) < f.len_b) write_seg(f.ring, i, first[i], lane);
    if constexpr (NSEG == kSlots) pend = first[kSlots - 1];
    f.dest = kSlots - 1;
    f.pend_new = 0u;
}

// Start of a stage.  The next segment's slot is free once every word of the
// segment kSlots earlier in the stream has been handed out.  Then the
// pending segment (the last one fetched), unless it is in the ring already,
// is written to its slot, and the next segment, when the stream has it, is
// fetched into the pending registers.  A fetched segment waits in registers
// until the next stage whose slot is free: its load has a stage or more to
// arrive, and the lanes, which take at most kChecksPerStage * 64 words per
// stage, reach its first word no earlier than the stage after that one.
__device__ __forceinline__ void feed_stage(Feed& f, Seg& pend, int lane) {
    static_assert(kDelay == 1, "one pending segment per stream");
    if (f.next_b <= 4u * f.handed + (uint32_t)((kSlots - 1) * kSegWords * 4)) {   // wave-uniform
        if (f.pend_new) write_seg(f.ring, f.dest, pend, lane);
        f.pend_new = 0u;
        if (f.next_b < f.len_b) {
            f.pend_new = 1u;
            pend = fetch_seg(f, f.next_b, lane);
            f.dest = f.next_slot;
            f.next_b += (uint32_t)(kSegWords * 4);
            f.next_slot = f.next_slot == (uint32_t)(kSlots - 1) ? 0u : f.next_slot + 1;
        }
    }
}

// A lane mask of the wave (one bit per lane, held in an SGPR pair).
typedef uint64_t Mask;

// x += y with the carry out of every lane as a lane mask (v_add_co_u32 with
// an SGPR carry).  Written out because the compiler turns the carry of an
// overflow add into a 0/1 VGPR and compares it again before a ballot.
__device__ __forceinline__ Mask add_carry(uint32_t& x, uint32_t y) {
    Mask c;
    asm("v_add_co_u32 %0, %1, %2, %3" : "=v"(x), "=s"(c) : "v"(x), "v"(y));
    return c;
}

// m's lanes take if_set, the others if_clear (v_cndmask_b32 on the mask).
__device__ __forceinline__ uint32_t select(Mask m, uint32_t if_set, uint32_t if_clear) {
    return __builtin_amdgcn_inverse_ballot_w64(m) ? if_set : if_clear;
}

// Two tANS steps.  One funnel shift gives the 32 bits from pos (two steps
// read at most 24); each step is a ds_read_b64 of the entry, a bit-field
// extract of nb bits (the second at offset nb1) and a shift-add for the next
// entry's offset.  q advances by nb1 + nb2 in both of its copies with one
// add (word0 holds nb in bits 4:0 and 30:27): the add's carry out is set
// exactly when the low window word is used up.  Returns the carry mask;
// w1/w2 get the two entries' word0.
__device__ __forceinline__ Mask dec_pair(Lane& l, const v2u* __restrict__ tbl, uint32_t& w1,
                                         uint32_t& w2) {
    const uint32_t t = __builtin_amdgcn_alignbit(l.hi, l.lo, l.q);   // shift = q[4:0]
    const v2u e1 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b1 = __builtin_amdgcn_ubfe(t, 0u, e1.x);           // width = nb1
    l.x8 = (b1 << 3) + e1.y;
    const v2u e2 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b2 = __builtin_amdgcn_ubfe(t, e1.x, e2.x);          // offset nb1, width nb2
    l.x8 = (b2 << 3) + e2.y;
    w1 = e1.x;
    w2 = e2.x;
    return add_carry(l.q, e1.x + e2.x);
}

// Three tANS steps from one funnel shift (tables of 2^11 states, nb <= 10:
// at most 30 bits).  The third step's field starts at nb1 + nb2, the low
// bits of word0_1 + word0_2 (at most 20, so the exponent bits above them
// are untouched); q advances by nb1 + nb2 + nb3 < 32 in both copies.
__device__ __forceinline__ Mask dec_triple(Lane& l, const v2u* __restrict__ tbl, uint32_t& w1,
                                           uint32_t& w2, uint32_t& w3) {
    const uint32_t t = __builtin_amdgcn_alignbit(l.hi, l.lo, l.q);   // shift = q[4:0]
    const v2u e1 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b1 = __builtin_amdgcn_ubfe(t, 0u, e1.x);           // width = nb1
    l.x8 = (b1 << 3) + e1.y;
    const v2u e2 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b2 = __builtin_amdgcn_ubfe(t, e1.x, e2.x);          // offset nb1, width nb2
    l.x8 = (b2 << 3) + e2.y;
    const uint32_t s12 = e1.x + e2.x;
    const v2u e3 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b3 = __builtin_amdgcn_ubfe(t, s12, e3.x);           // offset nb1 + nb2
    l.x8 = (b3 << 3) + e3.y;
    w1 = e1.x;
    w2 = e2.x;
    w3 = e3.x;
    return add_carry(l.q, s12 + e3.x);
}

// (c << 2) + b in one SALU instruction (s_lshl2_add_u32, which sets SCC).
__device__ __forceinline__ uint32_t lshl2_add(uint32_t c, uint32_t b) {
    uint32_t d;
    asm("s_lshl2_add_u32 %0, %1, %2" : "=s"(d) : "s"(c), "s"(b) : "scc");
    return d;
}

// Lanes in `need` take the next words of the stream in lane order (mbcnt
// rank, one ds_read_b32 from the ring); lanes in `shift` (a superset) move
// hi into lo.  Every lane reads the ring (in bounds: the mirror covers the
// 64 words past the ring end), so there is no divergent branch.  The mbcnt
// accumulator adds the ring's word index to the rank, so the read address
// is one shift-add of the rank and the wave's ring offset.  lds0 is the
// start of the workgroup's LDS.
__device__ __forceinline__ void refill(Lane& l, Feed& f, const void* lds0, Mask shift,
                                       Mask need) {
    const uint32_t idx = __builtin_amdgcn_mbcnt_hi((uint32_t)(need >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)need,
                                                                             f.ring_w));
    const uint32_t w = *reinterpret_cast<const uint32_t*>(
        reinterpret_cast<const char*>(lds0) + f.ring_b + idx * 4u);
    l.lo = select(shift, l.hi, l.lo);
    l.hi = select(need, w, l.hi);
    const uint32_t c = (uint32_t)__popcll(need);
    f.handed += c;
    const uint32_t nb = lshl2_add(c, f.ring_b);
    const uint32_t wrapped = nb - (uint32_t)(kRingWords * 4);
    f.ring_b = nb < wrapped ? nb : wrapped;   // (nb mod ring size), as an unsigned min
}

// The refill check after a segment of steps (`carry` from dec_pair or
// dec_triple; lanes out of range never carry, see lane_init): a lane whose
// low window word is used up (at most 32 unread bits) shifts and takes the
// next word.  There is no check after a stream's last segment, and in the
// last tile the checks go through check_last.
__device__ __forceinline__ void check(Lane& l, Feed& f, const void* lds0, Mask carry) {
    refill(l, f, lds0, carry, carry);
}

// check() in the last tile, with its kind chosen at run time (wave-uniform
// flags selecting lane masks): none after the stream's last segment; after
// the second-to-last one (final_check) a lane still shifts but takes a
// word only when it holds fewer bits than the last segment can read, that
// is when pos > fin_pos after the shift (fin_pos = 32 - that many bits:
// 8 for the pair schedule's 24).
__device__ __forceinline__ void check_last(Lane& l, Feed& f, const void* lds0, Mask carry,
                                           bool final_check, bool none, uint32_t fin_pos) {
    const Mask short_of_last = __ballot((l.q & 31u) > fin_pos);
    const Mask shift = none ? Mask(0) : carry;
    refill(l, f, lds0, shift, final_check ? shift & short_of_last : shift);
}

// Start a chain (after feed_commit): every lane in range takes two words,
// the first `lanes` stream words being the lanes' first words and the next
// `lanes` their second; pos = 0.  A lane out of range starts on the sink
// entry (byte offset `sink` from the table), whose steps read no bits and
// return to it, so its pos never moves and its refill checks never fire.
__device__ __forceinline__ void lane_init(Lane& l, Feed& f, int lane, int lanes, uint16_t state,
                                          uint32_t L, uint32_t sink) {
    const bool active = lane < lanes;
    const uint32_t* r = f.ring;
    l.lo = active ? r[lane] : 0u;
    l.hi = active ? r[lanes + lane] : 0u;
    l.q = 0;
    l.x8 = active ? ((uint32_t)(state - L) & (L - 1)) * 8u : sink;
    f.handed = 2u * (uint32_t)lanes;
    f.ring_b = 8u * (uint32_t)lanes;
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

// The decode table is copied into LDS by the kDecBlock threads of a
// decoder workgroup in two halves: table_fetch issues every load of the
// thread, table_store writes them once they arrive.  Entries that would
// step outside the table (nb > log2L or base + 2^nb > 2L), or read more
// bits than the refill schedule allows (nb > 10 in a 2^11-state table), are
// replaced by a harmless one, so a malformed table gives wrong bytes, never
// an out-of-range LDS access.
template <uint32_t L>
struct TableRegs {
    static_assert(L % kDecBlock == 0, "the table is split evenly over the workgroup");
    v2u e[L / kDecBlock];
};

template <uint32_t L>
__device__ __forceinline__ void table_fetch(TableRegs<L>& r, const v2u* __restrict__ table) {
    #pragma unroll
    for (uint32_t k = 0; k < L / kDecBlock; k++) r.e[k] = table[threadIdx.x + k * kDecBlock];
}

// PACKED: the entries of the packed-layout decoders, whose word0 keeps nb
// in bits 4:0 and moves the two exponents 8 bits up (bits 22:19 and
// 30:27), so that bits 15:0 of a sum of word0s are the sum of their nb.
template <uint32_t L, bool PACKED = false>
__device__ __forceinline__ void table_store(v2u* lds, const TableRegs<L>& r) {
    constexpr uint32_t log2L = 31 - __builtin_clz(L);
    constexpr uint32_t max_nb =
        log2L == tans_sched::kTripleLog2L ? tans_sched::kTripleMaxNb : log2L;
    #pragma unroll
    for (uint32_t k = 0; k < L / kDecBlock; k++) {
        v2u e = r.e[k];
        const uint32_t nb = e.x & 0xFFu;
        const uint32_t base = e.y >> 3;
        if (nb > max_nb || (e.x >> 27) != nb || (e.y & 7u) || base + (1u << nb) > L)
            e = v2u{e.x & 0x07FFFF00u, 0u};
        if constexpr (PACKED) e.x = (e.x & 0x1Fu) | ((e.x & 0x007FF800u) << 8);
        lds[threadIdx.x + k * kDecBlock] = e;
    }
}

// ---------------------------------------------------------------------
// Packed layout of short streams (include/tans_amd.h; schedule.h,
// tans_pack): pair alphabet, at most four 16-element tiles per lane.  A
// wave loads a group's whole stream (header of lane-pair bit counts, then
// the bit area) into its ring region with 16-byte loads, scans the counts
// once, and from then on each lane reads its own bits at a cursor: there
// is no shared word stream, no refill and no state array.  Even lanes read
// forwards from their pair's start, odd lanes backwards from its end.  Per
// two steps a lane takes the 32 bits at its cursor (one ds_read2_b32 and a
// funnel shift; odd lanes reverse them with v_bfrev), extracts the two
// fields as the streaming decoder does, and advances the cursor by nb1 +
// nb2 with one add of the two entries' word0 (table_store<L, true>).
// Kernels select it with FIRST = -(tiles per lane).
// ---------------------------------------------------------------------
constexpr int kPackRegionBytes = kRingAlloc * 4;
constexpr int kPackMaxSegs = 4;                 // 16-byte loads per lane for 4 tiles
static_assert(tans_pack::max_stream_bytes(tans_pack::kMaxSteps) + 8 <= kPackRegionBytes &&
                  kPackRegionBytes <= kPackMaxSegs * kSegWords * 4,
              "a packed stream of four tiles fits the ring region with 8 bytes to spare");

// Segment loads that cover a packed stream of NT tiles (8 NT pair steps).
__host__ __device__ constexpr int pack_segs(int NT) {
    return (int)((tans_pack::max_stream_bytes(8 * NT) + kSegWords * 4 - 1) / (kSegWords * 4));
}

// Odd lanes of the wave (the backward half of each lane pair).
constexpr Mask kOddLanes = 0xAAAAAAAAAAAAAAAAull;

struct PLane {
    uint32_t a;       // the window's start at c = 0: the pair start (even lanes),
                      // the pair end - 64 (odd lanes)
    uint32_t sgn;     // 1 (even lanes) or 0xFFFF (odd lanes)
    uint32_t c;       // bits 15:0 the lane's bits read so far; the bits above collect exponents
    uint32_t x8;      // (state - L) * 8
    uint32_t lo, hi;  // the first window of a stream (pk_start): 64 bits in decode order
};

// The 64 bits at the lane's cursor in decode order, as (hi:lo): area bits
// [p, p + 64) with p = a + c (even lanes), or a - c (odd lanes, whose bits
// run backwards: both words reversed and swapped), p taken mod 2^16 by
// v_mad_u32_u16 (c.u16 * sgn.u16 + a).  Three LDS words per lane.
__device__ __forceinline__ void pk_window(const PLane& l, const uint32_t* region, uint32_t& lo,
                                          uint32_t& hi) {
    uint32_t pos;
    asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(pos) : "v"(l.c), "v"(l.sgn), "v"(l.a));
    const uint32_t idx = __builtin_amdgcn_ubfe(pos, 5u, 11u);
    const uint32_t d0 = region[idx], d1 = region[idx + 1], d2 = region[idx + 2];
    const uint32_t w0 = __builtin_amdgcn_alignbit(d1, d0, pos);
    const uint32_t w1 = __builtin_amdgcn_alignbit(d2, d1, pos);
    lo = select(kOddLanes, __builtin_bitreverse32(w1), w0);
    hi = select(kOddLanes, __builtin_bitreverse32(w0), w1);
}

// Two tANS steps from the 32 bits t; w1/w2 get the entries' word0.
__device__ __forceinline__ void pk_steps(PLane& l, uint32_t t, const v2u* __restrict__ tbl,
                                         uint32_t& w1, uint32_t& w2) {
    const v2u e1 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b1 = __builtin_amdgcn_ubfe(t, 0u, e1.x);
    l.x8 = (b1 << 3) + e1.y;
    const v2u e2 = *reinterpret_cast<const v2u*>(reinterpret_cast<const char*>(tbl) + l.x8);
    const uint32_t b2 = __builtin_amdgcn_ubfe(t, e1.x, e2.x);
    l.x8 = (b2 << 3) + e2.y;
    w1 = e1.x;
    w2 = e2.x;
}

// A group's packed stream (words s .. e of comp, clamped to the buffer):
// NSEG 16-byte loads per lane, zeros past the stream.  Returns its bytes.
template <int NSEG>
__device__ __forceinline__ uint32_t pk_fetch(const uint32_t* comp, int64_t words, int64_t s,
                                             int64_t e, int lane, Seg (&seg)[kPackMaxSegs]) {
    s = s < 0 ? 0 : (s > words ? words : s);
    e = e < s ? s : (e > words ? words : e);
    const int64_t room = (words - s) * 4;
    const uint32_t bound = room > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)room;
    const int64_t len = (e - s) * 4;
    const uint32_t len_b = len > (int64_t)bound ? bound : (uint32_t)len;
    const Rsrc src = rsrc(comp + s, bound);
    #pragma unroll
    for (int i = 0; i < NSEG; i++) {
        const uint32_t b = (uint32_t)(i * kSegWords * 4);
        seg[i] = __builtin_amdgcn_raw_buffer_load_b128(src, b < len_b ? (uint32_t)lane * 16u + b
                                                                      : kNoSeg, 0, 0);
    }
    return len_b;
}

// Inclusive sum over the wave's lanes (DPP: four row shifts within each row
// of 16 lanes, then two row broadcasts across rows).
__device__ __forceinline__ uint32_t wave_scan(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);   // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);   // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);   // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);   // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return v;
}

// Write the stream into the wave's region (the fourth load only up to the
// region's end), read the header, set up the lane's cursor and take its
// first window: the state (12 bits) and the first two segments.  The
// wave's LDS accesses execute in order, so its reads see its writes.
// Cursors are clamped so that 8 NT steps (at most T bits) and the 96-bit
// read stay inside the region whatever the header says; a well-formed
// stream never meets the clamp.
template <int NT, int NSEG>
__device__ __forceinline__ void pk_start(PLane& l, uint32_t* region, int lane,
                                         const Seg (&seg)[kPackMaxSegs], uint32_t len_b) {
    // (compiler barriers: the region is written as 16-byte vectors and read
    // as words, which type-based alias analysis would let it reorder)
    asm volatile("" ::: "memory");
    #pragma unroll
    for (int i = 0; i < NSEG; i++)
        if ((i == 0 || (uint32_t)(i * kSegWords * 4) < len_b) &&
            ((i + 1) * kSegWords * 4 <= kPackRegionBytes ||
             lane * 16 < kPackRegionBytes - i * kSegWords * 4))
            reinterpret_cast<Seg*>(region + i * kSegWords)[lane] = seg[i];
    asm volatile("" ::: "memory");
    constexpr int hb = NT == 1 ? 1 : 2;   // tans_pack::hdr_bytes(8 NT)
    static_assert(hb == tans_pack::hdr_bytes(8 * NT) && hb == tans_pack::hdr_bytes(8 * NT - 7),
                  "one header width for every stream length of NT tiles");
    const uint32_t hbyte = (uint32_t)(lane >> 1) * hb;   // the pair's count in the header
    const uint32_t cnt = (region[hbyte >> 2] >> (8 * (hbyte & 3))) & (hb == 1 ? 0xFFu : 0xFFFFu);
    // the pair's end: the counts of even lanes summed up to this lane
    const uint32_t end = (uint32_t)tans_pack::hdr_total(8 * NT) * 8u +
                         wave_scan((lane & 1) ? 0u : cnt);
    constexpr uint32_t T = (uint32_t)tans_pack::max_lane_bits(8 * NT);
    constexpr uint32_t R = kPackRegionBytes * 8;
    if (lane & 1) {
        const uint32_t a = end - 64u;
        l.a = a < T ? T : (a > R - 96u ? R - 96u : a);
        l.sgn = 0xFFFFu;
    } else {
        const uint32_t a = end - cnt;
        l.a = a > R - 96u - T ? R - 96u - T : a;
        l.sgn = 1u;
    }
    l.c = 0u;
    pk_window(l, region, l.lo, l.hi);
    l.x8 = (l.lo & 0xFFFu) << 3;
}

// The 16 elements of one tile of every chain (4 exponent words each): two
// windows of two segments each.  START: the stream's first tile, whose
// first window is pk_start's, after the 12 bits of the state.
template <int C, bool START>
__device__ __forceinline__ void pk_tile(PLane (&l)[C], uint32_t* const (&region)[C],
                                        const v2u* __restrict__ tbl, uint32_t (&ex)[C][4]) {
    #pragma unroll
    for (int h = 0; h < 2; h++) {
        #pragma unroll
        for (int c = 0; c < C; c++) {
            uint32_t lo, hi, off = 0, w1, w2, w3, w4;
            if (START && h == 0) {
                lo = l[c].lo;
                hi = l[c].hi;
                off = (uint32_t)tans_pack::kStateBits;
            } else {
                pk_window(l[c], region[c], lo, hi);
            }
            pk_steps(l[c], __builtin_amdgcn_alignbit(hi, lo, off), tbl, w1, w2);
            const uint32_t s12 = off + w1 + w2;   // bits 15:0: off + nb1 + nb2
            uint32_t t2;
            if (START && h == 0) {   // 12 + nb1 + nb2 can reach 36: a 64-bit shift
                t2 = (uint32_t)((((uint64_t)hi << 32) | lo) >> (s12 & 63u));
            } else {                 // nb1 + nb2 <= 24
                t2 = __builtin_amdgcn_alignbit(hi, lo, s12);
            }
            pk_steps(l[c], t2, tbl, w3, w4);
            l[c].c += s12 + w3 + w4;
            ex[c][2 * h] = __builtin_amdgcn_perm(w2, w1, 0x07060302u);       // bytes 2, 3 of each
            ex[c][2 * h + 1] = __builtin_amdgcn_perm(w4, w3, 0x07060302u);
        }
    }
}

template <int SPS>
struct Alpha {
    static constexpr uint32_t L = SPS == 2 ? (1u << TANS_PAIR_LOG2L) : (1u << TANS_NIBBLE_LOG2L);
    static constexpr int kStagesPerTile = SPS == 2 ? 1 : 2;   // a stage is 8 steps
    // refill schedule (schedule.h): segments of 2 steps, or 3, 3, 2 per stage
    static constexpr bool kTriple = SPS == 1;
    static_assert(kTriple == ((31 - __builtin_clz(L)) == tans_sched::kTripleLog2L),
                  "the nibble alphabet's tables are the 3-3-2 schedule's");
    static constexpr int kSegsPerStage = kTriple ? 3 : 4;
    static constexpr int kSegsPerTile = kSegsPerStage * kStagesPerTile;
    static constexpr int seg_first(int q) { return kTriple ? 3 * q : 2 * q; }
    static constexpr int seg_len(int q) { return kTriple ? (q == 2 ? 2 : 3) : 2; }
    // the final check's fin_pos when the stream ends with a whole tile
    static constexpr uint32_t kFinPosFullTile =
        32u - (uint32_t)(kTriple ? tans_sched::kTripleMaxNb * 2 : tans_sched::kPairFinalBelow);
    // ring segments that hold a whole one-tile stream: under the refill
    // schedule a lane takes at most 3 words over 8 pair steps (768 bytes per
    // group) and at most 5 over 16 nibble steps (1280 bytes)
    static constexpr int kOneTileSegs = kTriple ? 2 : 1;
    // the most tiles whose streams fit the ring's kSlots segments: a lane
    // takes at most 12 words over 32 pair steps (3072 bytes per group) and
    // at most 10 over 32 nibble steps (2560 bytes)
    static constexpr int kResidentTiles = kTriple ? 2 : 4;
};

// Segments of S steps in the last tile and the final check's fin_pos
// (check_last), for a stream of n_tiles tiles.  When the last tile holds a
// single segment, the final check follows the last segment of the tile
// before, and the schedule makes it the plain check there (schedule.h), so
// every tile but the last takes the plain path.
template <int SPS>
__device__ __forceinline__ void last_tile_sched(int64_t S, int n_tiles, int& last_segs,
                                                uint32_t& fin_pos) {
    constexpr bool tri = Alpha<SPS>::kTriple;
    last_segs = (int)(tans_sched::segments(S, tri) -
                      (int64_t)(n_tiles - 1) * Alpha<SPS>::kSegsPerTile);
    fin_pos = S > 0 ? 32u - (uint32_t)tans_sched::final_below(S, tri) : 0u;
}

// LDS of a decoder workgroup.  The table comes first so that its entries'
// byte offsets are their LDS addresses.
template <int SPS, int C>
struct DecSmem {
    v2u tbl[Alpha<SPS>::L];
    uint32_t rings[kDecWaves][C][kRingAlloc];
    uint32_t progress;   // tiles finished by all waves of the workgroup
    v2u sink;            // the table entry of lanes out of range (lane_init)

    // The sink's byte offset from the table.
    __device__ __forceinline__ uint32_t sink_off() const {
        return (uint32_t)(reinterpret_cast<const char*>(&sink) -
                          reinterpret_cast<const char*>(tbl));
    }
    // By one thread before the workgroup's first barrier.  The sink reads
    // no bits (word0 = 0: nb = 0, exponents 0) and leads back to itself.
    __device__ __forceinline__ void init() {
        progress = 0;
        sink = v2u{0u, sink_off()};
    }
};

// Keep the waves of a workgroup abreast.  The SIMD arbiter prefers older
// waves, so without this the first wave on a SIMD finishes its groups in
// about half the time of the last, which then runs alone at a fraction of
// the SIMD's throughput.  After each tile a wave adds one to the
// workgroup's progress count and sets its priority from where it stands: a
// wave more than a tile ahead of the average yields (it still issues when
// the others stall), a wave behind the average goes first.
__device__ __forceinline__ void pace(uint32_t* progress, int lane, uint32_t done, uint32_t live) {
    uint32_t before = 0;
    if (lane == 0) before = __hip_atomic_fetch_add(progress, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP);
    before = __builtin_amdgcn_readfirstlane(before);
    const uint32_t mine = done * live;   // compare done with before / live
    __builtin_amdgcn_s_setprio(1);
    if (mine > before + 2 * live) __builtin_amdgcn_s_setprio(0);
    if (mine + live <= before) __builtin_amdgcn_s_setprio(3);
}

// C independent chains (a chain = one group's stream) decoded in lockstep
// by one wave, so each lane interleaves C serial tANS states.
template <int C>
struct Chains {
    Feed f[C];
    Lane l[C];
    Seg p[C];   // each chain's pending segment
};

// Decode the 16 elements of one tile of every chain into exponent words
// ex[c][4] (4 elements each).  q's scratch bits are cleared first (a
// segment adds less than 2^24 there).  LAST: the tile holds each stream's
// final segments, last_segs of them (the rest of the tile decodes past the
// end: no checks there, so it reads only the lane's own window and the
// table, and its bytes are discarded); fin_pos sets the final check
// (check_last).  RESIDENT: the streams were loaded whole at their start
// (feed_commit<NSEG>), so no stage fetches.
template <int SPS, int C, bool LAST, bool RESIDENT = false>
__device__ __forceinline__ void dec_tile(Chains<C>& ch, const v2u* __restrict__ tbl, int lane,
                                         uint32_t (&ex)[C][4],
                                         int last_segs = Alpha<SPS>::kSegsPerTile,
                                         uint32_t fin_pos = Alpha<SPS>::kFinPosFullTile) {
    using A = Alpha<SPS>;
    #pragma unroll
    for (int c = 0; c < C; c++) ch.l[c].q &= 0xF800001Fu;
    static_for<0, A::kStagesPerTile>([&](auto H) {
        constexpr int h = decltype(H)::value;
        if constexpr (!RESIDENT) {
            #pragma unroll
            for (int c = 0; c < C; c++) feed_stage(ch.f[c], ch.p[c], lane);
        }
        uint32_t e[C][8];
        static_for<0, A::kSegsPerStage>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            constexpr int i0 = A::seg_first(q);
            Mask carry[C];
            #pragma unroll
            for (int c = 0; c < C; c++) {
                if constexpr (A::seg_len(q) == 3)
                    carry[c] = dec_triple(ch.l[c], tbl, e[c][i0], e[c][i0 + 1], e[c][i0 + 2]);
                else
                    carry[c] = dec_pair(ch.l[c], tbl, e[c][i0], e[c][i0 + 1]);
            }
            if (LAST) {
                // the segment's index in the tile: segments from last_segs - 1
                // on end the streams (no check) and the one before them gets
                // the final check; selected on the masks, without branches
                const int idx = h * A::kSegsPerStage + q;
                #pragma unroll
                for (int c = 0; c < C; c++)
                    check_last(ch.l[c], ch.f[c], tbl, carry[c],
                               tans_sched::end_is_final(last_segs, idx),
                               tans_sched::end_is_none(last_segs, idx), fin_pos);
            } else {
                #pragma unroll
                for (int c = 0; c < C; c++) check(ch.l[c], ch.f[c], tbl, carry[c]);
            }
        });
        #pragma unroll
        for (int c = 0; c < C; c++) {
            if constexpr (SPS == 2) {
                #pragma unroll
                for (int i = 0; i < 4; i++) ex[c][i] = exp4_pair(e[c][2 * i], e[c][2 * i + 1]);
            } else {
                ex[c][2 * h] = exp4_nib(e[c][0], e[c][1], e[c][2], e[c][3]);
                ex[c][2 * h + 1] = exp4_nib(e[c][4], e[c][5], e[c][6], e[c][7]);
            }
        }
    });
}

// ---------------------------------------------------------------------
// Fused decode + add.  A wave decodes G groups of A and the same G groups
// of B (C = 2G chains) and writes their sums, tiled [N/16, K, 16].  The
// grid holds at most one workgroup per CU (the LDS allows no more), and a
// wave takes groups g, g + grid groups, ... in turn: the decode table is
// loaded once per CU, and short streams (down to one tile per lane) do not
// pay a workgroup launch and a table load per group.
// ---------------------------------------------------------------------
// FIRST > 0: every stream fits FIRST ring segments and is loaded whole at
// its start, with its (at most kSmAhead) sign/mantissa tiles: no stage
// fetches, no sign/mantissa prefetch.  FIRST = 0: streams of any length.
// FIRST < 0: the packed layout, -FIRST tiles per lane, loaded whole too.
template <int SPS, int G, int FIRST>
struct FusedWave {
    static constexpr bool PACKED = FIRST < 0;
    static constexpr bool RES = FIRST != 0;
    static constexpr int C = 2 * G;   // chain 2g: A of group g, 2g + 1: B of group g
    Chains<C> ch;
    PLane pk[C];            // packed layout: the lanes' cursors
    uint32_t* preg[C];      // packed layout: each chain's stream region (LDS)
    v2u sm[C][kSmAhead];    // sign/mantissa words of tiles t .. t + kSmAhead - 1 (by t mod kSmAhead)
    const char* pf[C];      // sign/mantissa row of the next prefetch (wave-uniform)
    char* out_cur[G];       // output row of the current tile (wave-uniform)
    uint32_t sm_bytes[G];   // bytes of a group's sm row (8 per lane in range)
    const v2u* tbl;
    uint32_t* progress;     // workgroup progress count (LDS)
    uint32_t live;          // waves of the workgroup with groups to decode
    int64_t sm_stride;      // bytes between tiles: K * 8
    int64_t out_stride;     // K * 16
    int n_tiles;
    int lane;
    int base;               // tiles this wave finished in earlier groups (pacing)

    // Tile t, with P = t mod kSmAhead; LAST: t is the last tile.
    template <int P, bool LAST>
    __device__ __forceinline__ void tile(int t) {
        uint32_t ex[C][4];
        if constexpr (PACKED) pk_tile<C, P == 0>(pk, preg, tbl, ex);
        else dec_tile<SPS, C, LAST, RES>(ch, tbl, lane, ex);
        pace(progress, lane, (uint32_t)(base + t), live);
        #pragma unroll
        for (int g = 0; g < G; g++) {
            uint32_t wa[4], wb[4];
            compose8(ex[2 * g][0], ex[2 * g][1], sm[2 * g][P].x, wa[0], wa[1]);
            compose8(ex[2 * g][2], ex[2 * g][3], sm[2 * g][P].y, wa[2], wa[3]);
            compose8(ex[2 * g + 1][0], ex[2 * g + 1][1], sm[2 * g + 1][P].x, wb[0], wb[1]);
            compose8(ex[2 * g + 1][2], ex[2 * g + 1][3], sm[2 * g + 1][P].y, wb[2], wb[3]);
            const v4u va = {wa[0], wa[1], wa[2], wa[3]};
            const v4u vb = {wb[0], wb[1], wb[2], wb[3]};
            __builtin_amdgcn_raw_buffer_store_b128(add16_fp8(va, vb),
                                                   rsrc(out_cur[g], sm_bytes[g] * 2u),
                                                   (uint32_t)lane * 16u, 0, kNT);
            out_cur[g] += out_stride;
        }
        // sign/mantissa of tile t + kSmAhead, when the stream has it.  Past the
        // last tile nothing is issued: a load with an empty bound reads nothing
        // but still takes its turn in the texture-address path, and with 8
        // tiles per stream half of a group's prefetches would be such loads
        // (skipping them: 128 per lane -2.5%, 1024 per lane -0.5%).
        if constexpr (RES) return;
        if (t + kSmAhead < n_tiles) {   // wave-uniform
            #pragma unroll
            for (int c = 0; c < C; c++)
                sm[c][P] = __builtin_amdgcn_raw_buffer_load_b64(
                    rsrc(pf[c], sm_bytes[c / 2]), (uint32_t)lane * 8u, 0, kNT);
        }
        if (t + kSmAhead + 1 < n_tiles) {
            #pragma unroll
            for (int c = 0; c < C; c++) pf[c] += sm_stride;
        }
    }
};

template <int SPS, int G, int FIRST>
__global__ __launch_bounds__(kDecBlock) void fused_add_kernel(
    const uint32_t* __restrict__ a_comp, int64_t a_words, const int64_t* __restrict__ a_off,
    const uint16_t* __restrict__ a_st, const v2u* __restrict__ a_sm,
    const uint32_t* __restrict__ b_comp, int64_t b_words, const int64_t* __restrict__ b_off,
    const uint16_t* __restrict__ b_st, const v2u* __restrict__ b_sm,
    const v2u* __restrict__ table, int64_t K, int n_tiles, v4u* __restrict__ out) {
    constexpr uint32_t L = Alpha<SPS>::L;
    constexpr int C = 2 * G;
    __shared__ DecSmem<SPS, C> smem;
    v2u* tbl = smem.tbl;
    // issue the table, stream, state and sign/mantissa loads together; a
    // wave past the last group loads the last one and leaves after the
    // barrier
    TableRegs<L> tr;
    table_fetch<L>(tr, table);
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t n_groups = (K + kLanes - 1) / kLanes;
    const int64_t grid_groups = (int64_t)gridDim.x * kDecWaves * G;   // groups per round
    int64_t g0 = ((int64_t)blockIdx.x * kDecWaves + wave) * G;
    const bool live = g0 < n_groups;   // wave-uniform
    const int64_t wg_groups = n_groups - (int64_t)blockIdx.x * kDecWaves * G;
    constexpr bool PACKED = FIRST < 0;
    // segments loaded at a start, and sign/mantissa tiles loaded then
    constexpr int NSEG = FIRST > 0 ? FIRST : PACKED ? pack_segs(-FIRST) : kSlots;
    constexpr int NSM = PACKED ? -FIRST : FIRST == Alpha<SPS>::kOneTileSegs ? 1 : kSmAhead;
    static_assert(FIRST == 0 || FIRST == Alpha<SPS>::kOneTileSegs || FIRST == kSlots ||
                      (PACKED && SPS == 2 && -FIRST <= kSmAhead),
                  "one-tile streams, streams of up to kResidentTiles tiles, any streams, or "
                  "packed streams of up to 4 tiles");
    static_assert(Alpha<SPS>::kResidentTiles <= kSmAhead,
                  "a resident stream's sign/mantissa tiles are all loaded at its start");
    FusedWave<SPS, G, FIRST> w;
    w.progress = &smem.progress;
    w.live = (uint32_t)(wg_groups >= (int64_t)kDecWaves * G ? kDecWaves : (wg_groups + G - 1) / G);
    w.lane = lane;
    w.n_tiles = n_tiles;
    w.tbl = tbl;
    w.sm_stride = K * 8;
    w.out_stride = K * 16;
    Seg first[C][PACKED ? kPackMaxSegs : kSlots];
    uint16_t st0[C];
    uint32_t plen[C];   // packed layout: bytes of each chain's stream
    int glanes[G];
    #pragma unroll
    for (int c = 0; c < C; c++) w.preg[c] = smem.rings[wave][c];
    // the loads of the groups gbase .. gbase + G - 1
    // With resident streams a wave switches groups every few tiles, and the
    // switch waits on the next group's stream offsets: they are loaded
    // during the last tile instead, by lanes 0-3 (a vector load, so the
    // tile's own waits do not include it), and read with v_readlane.
    // (not in the nibble kernel for two-tile streams: it has no VGPRs to spare)
    constexpr bool AHEAD = PACKED || (FIRST > 0 && (SPS == 2 || FIRST == Alpha<SPS>::kOneTileSegs));
    static_assert(G == 1 || !AHEAD, "offsets ahead for one group per wave");
    int64_t noff = 0;
    auto next_offsets = [&](int64_t gnext) {
        const int64_t g = gnext < n_groups ? gnext : n_groups - 1;
        if (lane < 4) noff = (lane < 2 ? a_off : b_off)[g + (lane & 1)];
    };
    auto noff_lane = [&](int l) {
        const uint32_t lo = (uint32_t)noff, hi = (uint32_t)((uint64_t)noff >> 32);
        return (int64_t)(((uint64_t)__builtin_amdgcn_readlane(hi, l) << 32) |
                         __builtin_amdgcn_readlane(lo, l));
    };
    auto setup = [&](int64_t gbase, bool ahead) {
        #pragma unroll
        for (int j = 0; j < G; j++) {
            // a wave past the last group repeats it with no lanes in range
            const int64_t g = gbase + j < n_groups ? gbase + j : n_groups - 1;
            const int64_t k0 = g * kLanes;
            const int lanes = gbase + j < n_groups ? (K - k0 < kLanes ? (int)(K - k0) : kLanes) : 0;
            const bool active = lane < lanes;
            const uint32_t lane_ld = (uint32_t)(active ? lane : (lanes ? lanes - 1 : 0));
            w.sm_bytes[j] = (uint32_t)lanes * 8u;
            w.out_cur[j] = reinterpret_cast<char*>(out + k0);
            int64_t sa, ea, sb, eb;
            if (ahead) {
                sa = noff_lane(0); ea = noff_lane(1); sb = noff_lane(2); eb = noff_lane(3);
            } else {
                sa = a_off[g]; ea = a_off[g + 1]; sb = b_off[g]; eb = b_off[g + 1];
            }
            if constexpr (PACKED) {
                plen[2 * j] = pk_fetch<NSEG>(a_comp, a_words, sa, ea, lane, first[2 * j]);
                plen[2 * j + 1] = pk_fetch<NSEG>(b_comp, b_words, sb, eb, lane, first[2 * j + 1]);
            } else {
                feed_fetch<NSEG>(w.ch.f[2 * j], a_comp, a_words, sa, ea, smem.rings[wave][2 * j],
                                 tbl, lane, first[2 * j]);
                feed_fetch<NSEG>(w.ch.f[2 * j + 1], b_comp, b_words, sb, eb,
                                 smem.rings[wave][2 * j + 1], tbl, lane, first[2 * j + 1]);
                st0[2 * j] = a_st[k0 + lane_ld];
                st0[2 * j + 1] = b_st[k0 + lane_ld];
            }
            glanes[j] = lanes;
            const char* rows[2] = {reinterpret_cast<const char*>(a_sm + k0),
                                   reinterpret_cast<const char*>(b_sm + k0)};
            #pragma unroll
            for (int s = 0; s < 2; s++) {
                const int c = 2 * j + s;
                #pragma unroll
                for (int i = 0; i < NSM; i++) {
                    const int64_t ti = i < n_tiles ? i : n_tiles - 1;
                    w.sm[c][i] = __builtin_amdgcn_raw_buffer_load_b64(
                        rsrc(rows[s] + ti * w.sm_stride, i < n_tiles ? w.sm_bytes[j] : 0u),
                        (uint32_t)lane * 8u, 0, kNT);
                }
                const int64_t tn = kSmAhead < n_tiles ? kSmAhead : n_tiles - 1;
                w.pf[c] = rows[s] + tn * w.sm_stride;
            }
        }
    };
    // Packed streams of one or two tiles: a wave switches groups every tile
    // or two, so the next group's stream and sign/mantissa tiles are loaded
    // as soon as the current stream is in LDS, before its tiles are decoded
    // (the offsets two groups ahead).  The loads are unconditional (a wave
    // past the last group loads that one again, to no use), so the waits of
    // the tiles in between count them exactly.
    constexpr bool PREFETCH = PACKED && -FIRST == 2;
    // One-tile streams take the streams two groups ahead (two stream
    // buffers in turn), the sign/mantissa tiles one group ahead.
    constexpr bool DEEP = PACKED && -FIRST == 1;
    v2u smn[C][(PREFETCH || DEEP) ? NSM : 1];   // the next group's sign/mantissa tiles
    uint32_t plen_n[C];               // and its streams' bytes
    auto prefetch = [&](int64_t gnext) {
        if constexpr (PREFETCH) {
            const int64_t g = gnext < n_groups ? gnext : n_groups - 1;
            const int64_t k0 = g * kLanes;
            const uint32_t smb = (uint32_t)(K - k0 < kLanes ? K - k0 : kLanes) * 8u;
            plen_n[0] = pk_fetch<NSEG>(a_comp, a_words, noff_lane(0), noff_lane(1), lane,
                                       first[0]);
            plen_n[1] = pk_fetch<NSEG>(b_comp, b_words, noff_lane(2), noff_lane(3), lane,
                                       first[1]);
            const char* rows[2] = {reinterpret_cast<const char*>(a_sm + k0),
                                   reinterpret_cast<const char*>(b_sm + k0)};
            #pragma unroll
            for (int c = 0; c < C; c++)
                #pragma unroll
                for (int i = 0; i < NSM; i++)
                    smn[c][i] = __builtin_amdgcn_raw_buffer_load_b64(
                        rsrc(rows[c] + (int64_t)i * w.sm_stride, smb), (uint32_t)lane * 8u, 0,
                        kNT);
        }
    };
    // the group after g0 becomes the current one (its loads were issued ahead)
    auto advance = [&]() {
        const int64_t k0 = g0 * kLanes;
        const int lanes = K - k0 < kLanes ? (int)(K - k0) : kLanes;
        w.sm_bytes[0] = (uint32_t)lanes * 8u;
        w.out_cur[0] = reinterpret_cast<char*>(out + k0);
        glanes[0] = lanes;
        #pragma unroll
        for (int c = 0; c < C; c++)
            #pragma unroll
            for (int i = 0; i < ((PREFETCH || DEEP) ? NSM : 1); i++) w.sm[c][i] = smn[c][i];
    };
    Seg second[C][DEEP ? kPackMaxSegs : 1];   // DEEP: the second stream buffer
    uint32_t plen2[C];
    setup(g0, false);
    if constexpr (PREFETCH) next_offsets(g0 + grid_groups);
    if constexpr (DEEP) {
        const int64_t g1 = g0 + grid_groups < n_groups ? g0 + grid_groups : n_groups - 1;
        plen2[0] = pk_fetch<NSEG>(a_comp, a_words, a_off[g1], a_off[g1 + 1], lane, second[0]);
        plen2[1] = pk_fetch<NSEG>(b_comp, b_words, b_off[g1], b_off[g1 + 1], lane, second[1]);
        next_offsets(g0 + 2 * grid_groups);
    }
    table_store<L, PACKED>(tbl, tr);
    if (threadIdx.x == 0) smem.init();
    __syncthreads();
    if (!live) return;
    int done = 0;   // tiles of earlier groups (the pacing count runs on)
    if constexpr (DEEP) {
        static_assert(G == 1, "one group per wave");
        // group g0's stream is in cur: put it in LDS, load group g0 + 2 grid's
        // into cur, then decode g0; false once the wave has no groups left
        auto step = [&](Seg (&cur)[C][DEEP ? kPackMaxSegs : 1], uint32_t (&pcur)[C]) -> bool {
            if constexpr (DEEP) {
                #pragma unroll
                for (int c = 0; c < C; c++)
                    pk_start<1, NSEG>(w.pk[c], w.preg[c], lane, cur[c], pcur[c]);
                pcur[0] = pk_fetch<NSEG>(a_comp, a_words, noff_lane(0), noff_lane(1), lane, cur[0]);
                pcur[1] = pk_fetch<NSEG>(b_comp, b_words, noff_lane(2), noff_lane(3), lane, cur[1]);
                next_offsets(g0 + 3 * grid_groups);
                const int64_t gn = g0 + grid_groups < n_groups ? g0 + grid_groups : n_groups - 1;
                const int64_t kn = gn * kLanes;
                const uint32_t smb = (uint32_t)(K - kn < kLanes ? K - kn : kLanes) * 8u;
                smn[0][0] = __builtin_amdgcn_raw_buffer_load_b64(
                    rsrc(reinterpret_cast<const char*>(a_sm + kn), smb), (uint32_t)lane * 8u, 0, kNT);
                smn[1][0] = __builtin_amdgcn_raw_buffer_load_b64(
                    rsrc(reinterpret_cast<const char*>(b_sm + kn), smb), (uint32_t)lane * 8u, 0, kNT);
                w.base = done;
                w.template tile<0, true>(0);
                done += 1;
                g0 += grid_groups;
                if (g0 >= n_groups) return false;
                advance();
            }
            return true;
        };
        for (;;) {
            if (!step(first, plen)) break;
            if (!step(second, plen2)) break;
        }
        return;
    }
    for (;;) {
        #pragma unroll
        for (int c = 0; c < C; c++) {
            if constexpr (PACKED) {
                pk_start<-FIRST, NSEG>(w.pk[c], w.preg[c], lane, first[c], plen[c]);
            } else {
                feed_commit<NSEG>(w.ch.f[c], lane, first[c], w.ch.p[c]);
                lane_init(w.ch.l[c], w.ch.f[c], lane, glanes[c / 2], st0[c], L, smem.sink_off());
            }
        }
        if constexpr (PREFETCH) {
            static_assert(G == 1, "one group per wave");
            prefetch(g0 + grid_groups);
            next_offsets(g0 + 2 * grid_groups);
        }
        w.base = done;
        // the first n_tiles - 1 tiles four per iteration, then the last one,
        // which ends the streams (its variant chosen by tile mod 4)
        const int body = n_tiles - 1;
        for (int t = 0; t < body; t += kSmAhead) {
            w.template tile<0, false>(t);
            if (t + 1 < body) w.template tile<1, false>(t + 1);
            if (t + 2 < body) w.template tile<2, false>(t + 2);
            if (t + 3 < body) w.template tile<3, false>(t + 3);
        }
        static_assert(kSmAhead == 4, "the loop above is unrolled for kSmAhead == 4");
        if constexpr (AHEAD && !PREFETCH) next_offsets(g0 + grid_groups);
        switch (body % kSmAhead) {
            case 0: w.template tile<0, true>(body); break;
            case 1: w.template tile<1, true>(body); break;
            case 2: w.template tile<2, true>(body); break;
            default: w.template tile<3, true>(body); break;
        }
        done += n_tiles;
        g0 += grid_groups;
        if (g0 >= n_groups) break;
        if constexpr (PREFETCH) {   // the group prefetched above becomes the current one
            advance();
            #pragma unroll
            for (int c = 0; c < C; c++) plen[c] = plen_n[c];
        } else {
            setup(g0, AHEAD);
        }
    }
}

// ---------------------------------------------------------------------
// Standalone decode: two adjacent groups of one tensor per wave (two
// independent chains per lane); output [N, K], element-major.  A wave takes
// group pairs g, g + grid groups, ... in turn (the launcher shrinks the grid
// to one workgroup per CU for columns of one or two tiles).
//
// A tile leaves each lane with 16 bytes of its own column (rows 16t ..
// 16t + 15).  A 4x4 byte transpose inside each quad of lanes (two DPP swaps
// and two v_perm per word) turns every word into 4 columns of one row.  When
// rows start 16-byte aligned (K % 16 == 0) and both groups are complete,
// the words of 8 rows go through LDS staging rows, and each lane stores 16
// consecutive columns of one row: every 8 lanes write a whole 128-byte line,
// non-temporally.  Otherwise each word is stored where it lands (4 rows x 64
// bytes per store instruction), and in a wave whose groups are not both
// complete (the tensor's last lanes) each store is checked against the
// lanes in range, down to single bytes.
// ---------------------------------------------------------------------
constexpr int kDecodeGroups = 2;

// Word d of lane i in a quad holds rows 4j..4j+3 of column i; the result
// holds columns 0..3 of row 4j+i.  sel1/sel2 are the lane's v_perm
// selectors (quad_selectors).
__device__ __forceinline__ uint32_t quad_transpose(uint32_t d, uint32_t sel1, uint32_t sel2) {
    // DPP quad_perm [2,3,0,1]: the word of lane i^2; [1,0,3,2]: of lane i^1
    const uint32_t x = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)d, 0x4E, 0xF, 0xF, false);
    d = __builtin_amdgcn_perm(x, d, sel1);
    const uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)d, 0xB1, 0xF, 0xF, false);
    return __builtin_amdgcn_perm(y, d, sel2);
}

// Step 1 keeps the lane's own half and takes the partner's (lanes 0,1:
// low halves; lanes 2,3: high halves); step 2 interleaves bytes the same way.
__device__ __forceinline__ void quad_selectors(int lane, uint32_t& sel1, uint32_t& sel2) {
    sel1 = (lane & 2) ? 0x03020706u : 0x05040100u;
    sel2 = (lane & 1) ? 0x03070105u : 0x06020400u;
}

// Row-major staging of 8 output rows x 128 columns per wave (the wave's two
// groups) for whole-line stores.  Rows are kXposeStride dwords apart: 48 is
// 16 mod 32, so the four rows a quad writes fall in alternating halves of
// the banks.  The last row needs no padding.
constexpr int kXposeStride = 48;
constexpr int kXposeWords = 7 * kXposeStride + kDecodeGroups * kLanes / 4;

template <int SPS>
struct DecodeSmem {
    DecSmem<SPS, kDecodeGroups> dec;
    alignas(16) uint32_t xpose[kDecWaves][kXposeWords];
};
static_assert(sizeof(DecodeSmem<2>) <= 160 * 1024 && sizeof(DecodeSmem<1>) <= 160 * 1024,
              "decoder LDS exceeds the 160 KiB of a gfx950 CU");

// FIRST as in FusedWave: > 0 for streams loaded whole at their start,
// < 0 for the packed layout.
template <int SPS, int FIRST>
struct DecodeWave {
    static constexpr int C = kDecodeGroups;
    static constexpr bool PACKED = FIRST < 0;
    static constexpr bool RES = FIRST != 0;
    Chains<C> ch;
    PLane pk[C];            // packed layout: the lanes' cursors
    uint32_t* preg[C];      // packed layout: each group's stream region (LDS)
    v2u sm[C][kSmAhead];    // sign/mantissa words of tiles t .. t + kSmAhead - 1 (by t mod kSmAhead)
    const char* pf[C];      // sign/mantissa row of the next prefetch (wave-uniform)
    uint32_t sm_bytes[C];   // bytes of a group's sm row (8 per lane in range)
    int lanes[C];           // lanes of each group in range
    uint8_t* out_tile;      // row 16t, column k0 (wave-uniform)
    const v2u* tbl;
    uint32_t* progress;
    uint32_t live;
    int64_t K;
    int64_t sm_stride;      // K * 8
    uint32_t qoff;          // (lane & 3) * K + (lane >> 2) * 4: the lane's word after the transpose
    uint32_t sel1, sel2;
    uint32_t* xp;           // this wave's staging rows (LDS)
    int n_tiles;
    int lane;
    int base;               // tiles this wave finished in earlier groups (pacing)
    bool full;              // both groups have 64 lanes in range (wave-uniform)
    bool lines;             // K % 16 == 0: rows start 16-byte aligned
    int last_segs;          // refill segments of the streams in the last tile
    uint32_t fin_pos;       // the final check's threshold (check_last)

    // Tile t (P = t mod kSmAhead) holding n elements per lane (n < 16 only
    // for a ragged last tile); LAST: t is the last tile.
    template <int P, bool LAST>
    __device__ __forceinline__ void tile(int t, int n) {
        // A ragged tile is decoded in full: the steps past the lane's last
        // symbol come after every real one (no refill checks there), stay
        // inside the table, and their bytes are not stored.
        uint32_t ex[C][4];
        if constexpr (PACKED) pk_tile<C, P == 0>(pk, preg, tbl, ex);
        else dec_tile<SPS, C, LAST, RES>(ch, tbl, lane, ex, last_segs, fin_pos);
        pace(progress, lane, (uint32_t)(base + t), live);
        uint32_t w[C][4];
        #pragma unroll
        for (int g = 0; g < C; g++) {
            compose8(ex[g][0], ex[g][1], sm[g][P].x, w[g][0], w[g][1]);
            compose8(ex[g][2], ex[g][3], sm[g][P].y, w[g][2], w[g][3]);
        }
        if (full && n == kTile && lines) {   // wave-uniform
            // rows 8h .. 8h + 7 of both groups go through the staging rows;
            // lane l then stores columns 16 (l & 7) .. + 15 of row 8h + l / 8,
            // so each 8 lanes write one whole 128-byte line (non-temporal).
            // The wave's LDS accesses execute in order, so the writes of
            // half h = 1 come after the reads of half 0.
            #pragma unroll
            for (int h = 0; h < 2; h++) {
                #pragma unroll
                for (int g = 0; g < C; g++) {
                    #pragma unroll
                    for (int jj = 0; jj < 2; jj++)
                        xp[(4 * jj + (lane & 3)) * kXposeStride + 16 * g + (lane >> 2)] =
                            quad_transpose(w[g][2 * h + jj], sel1, sel2);
                }
                const v4u v = *reinterpret_cast<const v4u*>(xp + (lane >> 3) * kXposeStride +
                                                            (lane & 7) * 4);
                __builtin_nontemporal_store(
                    v, reinterpret_cast<v4u*>(out_tile + (int64_t)(8 * h + (lane >> 3)) * K +
                                              (lane & 7) * 16));
            }
        } else if (full && n == kTile) {
            #pragma unroll
            for (int g = 0; g < C; g++) {
                #pragma unroll
                for (int j = 0; j < 4; j++)
                    *reinterpret_cast<uint32_t*>(out_tile + (int64_t)j * 4 * K + g * kLanes + qoff) =
                        quad_transpose(w[g][j], sel1, sel2);
            }
        } else {
            const int row_in_quad = lane & 3;
            #pragma unroll
            for (int g = 0; g < C; g++) {
                // columns of this lane's transposed words that are in range
                const int valid = lanes[g] - 4 * (lane >> 2);
                #pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t v = quad_transpose(w[g][j], sel1, sel2);
                    uint8_t* p = out_tile + (int64_t)j * 4 * K + g * kLanes + qoff;
                    if (4 * j + row_in_quad < n && valid > 0) {
                        if (valid >= 4) {
                            *reinterpret_cast<uint32_t*>(p) = v;
                        } else {
                            p[0] = (uint8_t)v;
                            if (valid > 1) p[1] = (uint8_t)(v >> 8);
                            if (valid > 2) p[2] = (uint8_t)(v >> 16);
                        }
                    }
                }
            }
        }
        out_tile += kTile * K;
        if constexpr (RES) return;   // every sign/mantissa tile was loaded at the start
        // sign/mantissa of tile t + kSmAhead, when the stream has it (past the
        // last tile nothing is issued, as in FusedWave::tile: 128 per lane
        // -3.5%)
        if (t + kSmAhead < n_tiles) {   // wave-uniform
            #pragma unroll
            for (int g = 0; g < C; g++)
                sm[g][P] = __builtin_amdgcn_raw_buffer_load_b64(rsrc(pf[g], sm_bytes[g]),
                                                                (uint32_t)lane * 8u, 0, kNT);
        }
        if (t + kSmAhead + 1 < n_tiles) {
            #pragma unroll
            for (int g = 0; g < C; g++) pf[g] += sm_stride;
        }
    }

    // All tiles: the first n_tiles - 1 four per iteration (the sign/mantissa
    // buffers rotate by four), then the last one, which holds n_last
    // elements and ends the streams.
    __device__ __forceinline__ void run(int n_last) {
        static_assert(kSmAhead == 4, "the loop below is unrolled for kSmAhead == 4");
        const int body = n_tiles - 1;
        for (int t = 0; t < body; t += kSmAhead) {
            tile<0, false>(t, kTile);
            if (t + 1 < body) tile<1, false>(t + 1, kTile);
            if (t + 2 < body) tile<2, false>(t + 2, kTile);
            if (t + 3 < body) tile<3, false>(t + 3, kTile);
        }
        switch (body % kSmAhead) {
            case 0: tile<0, true>(body, n_last); break;
            case 1: tile<1, true>(body, n_last); break;
            case 2: tile<2, true>(body, n_last); break;
            default: tile<3, true>(body, n_last); break;
        }
    }
};


template <int SPS, int FIRST>
__global__ __launch_bounds__(kDecBlock) void decode_kernel(
    const uint32_t* __restrict__ comp, int64_t words, const int64_t* __restrict__ off,
    const uint16_t* __restrict__ st, const v2u* __restrict__ sm,
    const v2u* __restrict__ table, int64_t K, int64_t N, uint8_t* __restrict__ out) {
    constexpr uint32_t L = Alpha<SPS>::L;
    constexpr int C = kDecodeGroups;
    __shared__ DecodeSmem<SPS> dsmem;
    DecSmem<SPS, C>& smem = dsmem.dec;
    v2u* tbl = smem.tbl;
    // loads issued together, as in fused_add_kernel
    TableRegs<L> tr;
    table_fetch<L>(tr, table);
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t n_groups = (K + kLanes - 1) / kLanes;
    const int64_t grid_groups = (int64_t)gridDim.x * kDecWaves * C;   // groups per round
    int64_t g0 = ((int64_t)blockIdx.x * kDecWaves + wave) * C;
    const bool live = g0 < n_groups;   // wave-uniform
    const int64_t wg_groups = n_groups - (int64_t)blockIdx.x * kDecWaves * C;
    // as in fused_add_kernel (a lazy start measured within noise here:
    // 2^30 elements at 1024 per lane -0.3%, at 128 per lane +0.6%)
    constexpr bool PACKED = FIRST < 0;
    constexpr int NSEG = FIRST > 0 ? FIRST : PACKED ? pack_segs(-FIRST) : kSlots;
    constexpr int NSM = PACKED ? -FIRST : FIRST == Alpha<SPS>::kOneTileSegs ? 1 : kSmAhead;
    static_assert(FIRST == 0 || FIRST == Alpha<SPS>::kOneTileSegs || FIRST == kSlots ||
                      (PACKED && SPS == 2 && -FIRST <= kSmAhead),
                  "one-tile streams, streams of up to kResidentTiles tiles, any streams, or "
                  "packed streams of up to 4 tiles");
    DecodeWave<SPS, FIRST> w;
    w.progress = &smem.progress;
    w.live = (uint32_t)(wg_groups >= (int64_t)kDecWaves * C ? kDecWaves : (wg_groups + C - 1) / C);
    w.lane = lane;
    w.K = K;
    const int rag = (int)(N % kTile);
    w.n_tiles = (int)(N / kTile) + (rag ? 1 : 0);
    last_tile_sched<SPS>(N / SPS, w.n_tiles, w.last_segs, w.fin_pos);
    w.tbl = tbl;
    w.sm_stride = K * 8;
    w.qoff = (uint32_t)(lane & 3) * (uint32_t)K + (uint32_t)(lane >> 2) * 4u;
    quad_selectors(lane, w.sel1, w.sel2);
    w.xp = dsmem.xpose[wave];
    w.lines = K % 16 == 0;
    Seg first[C][PACKED ? kPackMaxSegs : kSlots];
    uint16_t st0[C];
    uint32_t plen[C];   // packed layout: bytes of each group's stream
    #pragma unroll
    for (int j = 0; j < C; j++) w.preg[j] = smem.rings[wave][j];
    // the loads of the groups gbase, gbase + 1
    auto setup = [&](int64_t gbase) {
        bool full = true;
        w.out_tile = out + gbase * kLanes;
        // a wave past the last group repeats it with no lanes in range
        int64_t os[C], oe[C];
        #pragma unroll
        for (int j = 0; j < C; j++) {
            const int64_t g = gbase + j < n_groups ? gbase + j : n_groups - 1;
            os[j] = off[g];
            oe[j] = off[g + 1];
        }
        #pragma unroll
        for (int j = 0; j < C; j++) {
            const int64_t g = gbase + j < n_groups ? gbase + j : n_groups - 1;
            const int64_t k0 = g * kLanes;
            const int lanes = gbase + j < n_groups ? (K - k0 < kLanes ? (int)(K - k0) : kLanes) : 0;
            full = full && lanes == kLanes;
            w.lanes[j] = lanes;
            const bool active = lane < lanes;
            const uint32_t lane_ld = (uint32_t)(active ? lane : (lanes ? lanes - 1 : 0));
            w.sm_bytes[j] = (uint32_t)lanes * 8u;
            if constexpr (PACKED) {
                plen[j] = pk_fetch<NSEG>(comp, words, os[j], oe[j], lane, first[j]);
            } else {
                feed_fetch<NSEG>(w.ch.f[j], comp, words, os[j], oe[j], smem.rings[wave][j], tbl,
                                 lane, first[j]);
                st0[j] = st[k0 + lane_ld];
            }
            const char* row = reinterpret_cast<const char*>(sm + k0);
            #pragma unroll
            for (int i = 0; i < NSM; i++) {
                const int64_t ti = i < w.n_tiles ? i : w.n_tiles - 1;
                w.sm[j][i] = __builtin_amdgcn_raw_buffer_load_b64(
                    rsrc(row + ti * w.sm_stride, i < w.n_tiles ? w.sm_bytes[j] : 0u),
                    (uint32_t)lane * 8u, 0, kNT);
            }
            const int64_t tn = kSmAhead < w.n_tiles ? kSmAhead : w.n_tiles - 1;
            w.pf[j] = row + tn * w.sm_stride;
        }
        w.full = full;
    };
    setup(g0);
    table_store<L, PACKED>(tbl, tr);
    if (threadIdx.x == 0) smem.init();
    __syncthreads();
    if (!live) return;
    int done = 0;   // tiles of earlier groups (the pacing count runs on)
    for (;;) {
        #pragma unroll
        for (int j = 0; j < C; j++) {
            if constexpr (PACKED) {
                pk_start<-FIRST, NSEG>(w.pk[j], w.preg[j], lane, first[j], plen[j]);
            } else {
                feed_commit<NSEG>(w.ch.f[j], lane, first[j], w.ch.p[j]);
                lane_init(w.ch.l[j], w.ch.f[j], lane, w.lanes[j], st0[j], L, smem.sink_off());
            }
        }
        w.base = done;
        w.run(rag ? rag : kTile);
        done += w.n_tiles;
        g0 += grid_groups;
        if (g0 >= n_groups) break;
        setup(g0);
    }
}

// ---------------------------------------------------------------------
// Fused decode + skinny GEMM: y[b][r] = scale * sum_c W[r][c] * x[b][c]
// with W tANS-coded and B <= 8 rows of bf16 x, on the matrix cores.
//
// Encoding (rans_vectoradd.tans_codec.encode_matrix): W, padded to Rp rows
// (a multiple of 64) and S * Nc columns (Nc a multiple of 32), is cut into
// S column segments of Nc columns.  A group is 16 rows of one segment:
// lane j = 16 q + r holds row r of the group and, of every 64-column block
// of the segment, the 16 columns 16 q .. 16 q + 15 (a last block of 32
// columns: the 8 columns 8 q .. 8 q + 7).  So one tile of a lane (16
// elements) is exactly what v_mfma_f32_16x16x32_bf16 takes from that lane
// as its A operand, split in two k-blocks of 8: the wave's 64 lanes hold a
// 16-row x 64-column block of W.  x comes from an LDS stage of the
// segment's columns (zero past the segment or the matrix), as the B
// operand: lane j reads x[j % 16][the same 8 columns] (lanes j % 16 >= B
// read a row whose products are never stored).  The 4 fp32 accumulators of
// lane j hold rows 4 (j / 16) .. 4 (j / 16) + 3 of the group for batch row
// j % 16.  The batch size does not change the work per tile.
//
// A workgroup takes one segment and up to 32 row groups (two per wave, two
// chains per lane).  Partial sums go to a workspace [S][B][Rp] and
// gemm_finalize_kernel adds the S segments in a fixed order, scales and
// rounds to bf16 (round to nearest even).
// ---------------------------------------------------------------------
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kGemmChains = 2;                        // row groups per wave
constexpr int kGemmGroupRows = 16;                    // rows of a group
constexpr int kGemmGroupsPerBlock = kDecWaves * kGemmChains;
constexpr int kGemmMaxBatch = 8;
constexpr int kGemmMaxSegCols = 1024;                 // Nc limit
constexpr int kGemmXStride = kGemmMaxSegCols + 16;    // bf16 per x stage row (32 bytes of pad)
static_assert(kGemmMaxSegCols == kDecBlock, "one x stage column per thread");

template <int SPS>
struct GemmSmem {
    DecSmem<SPS, kGemmChains> dec;
    alignas(16) __bf16 xs[kGemmMaxBatch][kGemmXStride];   // x columns of the segment
};
static_assert(sizeof(GemmSmem<2>) <= 160 * 1024 && sizeof(GemmSmem<1>) <= 160 * 1024,
              "the GEMM workgroup's LDS fits one CU");

// Four bf16 pairs from 4 FP8 words (exact: every E4M3FN value is a bf16).
__device__ __forceinline__ v8bf fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
    const v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    const v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    const v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    const v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    return v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int SPS>
struct GemmWave {
    static constexpr int C = kGemmChains;
    Chains<C> ch;
    v2u sm[C][kSmAhead];
    const char* pf[C];
    uint32_t sm_bytes;
    const v2u* tbl;
    const __bf16* xrow;     // this lane's x stage row
    uint32_t* progress;
    uint32_t live;
    int64_t sm_stride;
    int n_tiles;
    int last_segs;          // refill segments of the streams in the last tile
    uint32_t fin_pos;       // the final check's threshold (check_last)
    int lane;
    int q;                  // lane / 16: the lane's column chunk
    v4f acc[C];

    template <int P, bool LAST>
    __device__ __forceinline__ void tile(int t, int n) {
        // a half last tile (n = 8) is decoded in full (see DecodeWave::tile)
        // and its bytes past n are zeroed; every lane of a group is in range
        // (rows are padded to 64)
        uint32_t ex[C][4];
        dec_tile<SPS, C, LAST>(ch, tbl, lane, ex, last_segs, fin_pos);
        pace(progress, lane, (uint32_t)t, live);
        // x of the lane's columns: 64 t + 16 q (+ 8 for the second k-block),
        // or 64 t + 8 q in a half tile
        const int col = 64 * t + (n < kTile ? 8 : 16) * q;
        const v8bf x0 = *reinterpret_cast<const v8bf*>(xrow + col);
        const v8bf x1 = *reinterpret_cast<const v8bf*>(xrow + col + 8);
        #pragma unroll
        for (int c = 0; c < C; c++) {
            uint32_t w[4];
            compose8(ex[c][0], ex[c][1], sm[c][P].x, w[0], w[1]);
            compose8(ex[c][2], ex[c][3], sm[c][P].y, w[2], w[3]);
            if (n < kTile) { w[2] = 0u; w[3] = 0u; }   // wave-uniform: only n = 8 occurs
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(w[0], w[1]), x0,
                                                              acc[c], 0, 0, 0);
            if (n == kTile)
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(w[2], w[3]), x1,
                                                                  acc[c], 0, 0, 0);
        }
        // sign/mantissa of tile t + kSmAhead, with an empty bound past the last
        // tile.  Here the loads stay unconditional: skipping them behind a
        // branch, as FusedWave::tile does, measured slower in this kernel (6
        // more VGPRs, +0.45 us per 17408 x 5120 call).
        const bool sm_next = t + kSmAhead < n_tiles;   // wave-uniform
        #pragma unroll
        for (int c = 0; c < C; c++)
            sm[c][P] = __builtin_amdgcn_raw_buffer_load_b64(
                rsrc(pf[c], sm_next ? sm_bytes : 0u), (uint32_t)lane * 8u, 0, kNT);
        if (t + kSmAhead + 1 < n_tiles) {
            #pragma unroll
            for (int c = 0; c < C; c++) pf[c] += sm_stride;
        }
    }

    // as DecodeWave::run
    __device__ __forceinline__ void run(int n_last) {
        static_assert(kSmAhead == 4, "the loop below is unrolled for kSmAhead == 4");
        const int body = n_tiles - 1;
        for (int t = 0; t < body; t += kSmAhead) {
            tile<0, false>(t, kTile);
            if (t + 1 < body) tile<1, false>(t + 1, kTile);
            if (t + 2 < body) tile<2, false>(t + 2, kTile);
            if (t + 3 < body) tile<3, false>(t + 3, kTile);
        }
        switch (body % kSmAhead) {
            case 0: tile<0, true>(body, n_last); break;
            case 1: tile<1, true>(body, n_last); break;
            case 2: tile<2, true>(body, n_last); break;
            default: tile<3, true>(body, n_last); break;
        }
    }
};

// Grid: S * row_blocks workgroups; block (s, rb) decodes row groups
// [32 rb, 32 rb + 32) of segment s (16 rows each).  R: rows, Rp: rows
// padded to 64, C: columns, Nc: columns per segment, NB: batch rows.
template <int SPS>
__global__ __launch_bounds__(kDecBlock) void gemm_fused_kernel(
    const uint32_t* __restrict__ comp, int64_t words, const int64_t* __restrict__ off,
    const uint16_t* __restrict__ st, const v2u* __restrict__ sm, const v2u* __restrict__ table,
    int64_t Rp, int64_t C, int S, int Nc, int row_blocks, const uint16_t* __restrict__ x, int NB,
    float* __restrict__ ws) {
    constexpr uint32_t L = Alpha<SPS>::L;
    constexpr int CH = kGemmChains;
    __shared__ GemmSmem<SPS> smem;
    const int s = (int)(blockIdx.x / (unsigned)row_blocks);
    const int rb = (int)(blockIdx.x % (unsigned)row_blocks);
    const int64_t n_rg = Rp / kGemmGroupRows;               // row groups per segment
    // issue the x, table, stream, state and sign/mantissa loads together
    // (as in fused_add_kernel); a wave past the last row group loads the
    // last one and leaves after the barrier.  Thread i stages column i of
    // the segment for every batch row (zero past the segment, the matrix
    // or the batch).
    const int xc = (int)threadIdx.x;
    const int64_t xcol = (int64_t)s * Nc + xc;
    const bool x_in = xc < Nc && xcol < C;
    uint16_t xv[kGemmMaxBatch];
    #pragma unroll
    for (int b = 0; b < kGemmMaxBatch; b++)
        xv[b] = (b < NB && x_in) ? x[(int64_t)b * C + xcol] : (uint16_t)0;
    TableRegs<L> tr;
    table_fetch<L>(tr, table);
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t rg0 = (int64_t)rb * kGemmGroupsPerBlock + (int64_t)wave * CH;
    const bool live = rg0 < n_rg;   // wave-uniform
    const int64_t rg_left = n_rg - (int64_t)rb * kGemmGroupsPerBlock;
    GemmWave<SPS> w;
    w.progress = &smem.dec.progress;
    w.live = (uint32_t)(rg_left >= kGemmGroupsPerBlock ? kDecWaves : (rg_left + CH - 1) / CH);
    w.lane = lane;
    w.q = lane >> 4;
    w.tbl = smem.dec.tbl;
    w.xrow = &smem.xs[lane & (kGemmMaxBatch - 1)][0];
    w.sm_stride = (int64_t)S * n_rg * kLanes * 8;            // lanes: S * n_rg * 64
    const int per_lane = Nc / 4;                              // elements per lane (8 | per_lane)
    const int rag = per_lane % kTile;                         // 0 or 8
    w.n_tiles = per_lane / kTile + (rag ? 1 : 0);
    last_tile_sched<SPS>(per_lane / SPS, w.n_tiles, w.last_segs, w.fin_pos);
    w.sm_bytes = kLanes * 8u;
    Seg first[CH][kSlots];
    uint16_t st0[CH];
    // a wave with one row group left repeats it as its second chain and
    // discards that chain's sums
    int64_t os[CH], oe[CH];
    #pragma unroll
    for (int j = 0; j < CH; j++) {
        const int64_t g = (int64_t)s * n_rg + (rg0 + j < n_rg ? rg0 + j : n_rg - 1);
        os[j] = off[g];
        oe[j] = off[g + 1];
    }
    #pragma unroll
    for (int j = 0; j < CH; j++) {
        const int64_t rg = rg0 + j < n_rg ? rg0 + j : n_rg - 1;
        const int64_t g = (int64_t)s * n_rg + rg;
        const int64_t k0 = g * kLanes;
        // a lazy start: the first burst of loads, which decoding waits for,
        // is a third smaller (17408 x 5120 at B = 1: 25.5 -> 24.7 us per call)
        feed_fetch<kLazySegs>(w.ch.f[j], comp, words, os[j], oe[j], smem.dec.rings[wave][j],
                              smem.dec.tbl, lane, first[j]);
        st0[j] = st[k0 + lane];
        const char* row = reinterpret_cast<const char*>(sm + k0);
        #pragma unroll
        for (int i = 0; i < kSmAhead; i++) {
            const int64_t ti = i < w.n_tiles ? i : w.n_tiles - 1;
            w.sm[j][i] = __builtin_amdgcn_raw_buffer_load_b64(
                rsrc(row + ti * w.sm_stride, i < w.n_tiles ? w.sm_bytes : 0u), (uint32_t)lane * 8u,
                0, kNT);
        }
        const int64_t tn = kSmAhead < w.n_tiles ? kSmAhead : w.n_tiles - 1;
        w.pf[j] = row + tn * w.sm_stride;
        w.acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
    #pragma unroll
    for (int b = 0; b < kGemmMaxBatch; b++)
        smem.xs[b][xc] = __builtin_bit_cast(__bf16, xv[b]);
    if (xc < kGemmXStride - kGemmMaxSegCols) {
        #pragma unroll
        for (int b = 0; b < kGemmMaxBatch; b++)
            smem.xs[b][kGemmMaxSegCols + xc] = __builtin_bit_cast(__bf16, (uint16_t)0);
    }
    table_store<L>(smem.dec.tbl, tr);
    if (threadIdx.x == 0) smem.dec.init();
    __syncthreads();
    if (!live) return;
    #pragma unroll
    for (int j = 0; j < CH; j++) {
        feed_commit<kLazySegs>(w.ch.f[j], lane, first[j], w.ch.p[j]);
        lane_init(w.ch.l[j], w.ch.f[j], lane, kLanes, st0[j], L, smem.dec.sink_off());
    }
    w.run(rag ? rag : kTile);
    const int bn = lane & 15;   // the batch row of this lane's sums
    if (bn >= NB) return;
    #pragma unroll
    for (int j = 0; j < CH; j++) {
        if (rg0 + j >= n_rg) break;
        const int64_t r = (rg0 + j) * kGemmGroupRows + 4 * w.q;
        *reinterpret_cast<v4f*>(ws + ((int64_t)s * NB + bn) * Rp + r) = w.acc[j];
    }
}

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);   // quiet NaN
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// y[b][r] = bf16(scale * sum over s of ws[s][b][r]).  A block of 4 waves
// takes 64 consecutive outputs of one batch row: wave w sums segments
// s = w, w + 4, ... in ascending order (coalesced 256-byte loads), and the
// four sums are added in wave order, so the result is deterministic.  A
// wave issues the loads of kFinBatch segments before it adds any of them,
// so a call pays one memory round trip per kFinBatch segments instead of
// one per segment.
constexpr int kFinWaves = 4;
constexpr int kFinBatch = 8;

__global__ __launch_bounds__(kFinWaves * kLanes) void gemm_finalize_kernel(
    const float* __restrict__ ws, int S, int NB, int64_t Rp, int64_t R, float scale,
    uint16_t* __restrict__ y) {
    __shared__ float part[kFinWaves][kLanes];
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = threadIdx.x / kLanes;
    const int64_t blocks_per_b = (R + kLanes - 1) / kLanes;
    const int64_t b = blockIdx.x / blocks_per_b;
    const int64_t r = (blockIdx.x % blocks_per_b) * kLanes + lane;   // < Rp: Rp is a multiple of 64
    float a = 0.0f;
    for (int s0 = wave; s0 < S; s0 += kFinWaves * kFinBatch) {
        float v[kFinBatch];
        #pragma unroll
        for (int i = 0; i < kFinBatch; i++) {
            const int s = s0 + i * kFinWaves < S ? s0 + i * kFinWaves : S - 1;   // in bounds
            v[i] = ws[((int64_t)s * NB + b) * Rp + r];
        }
        #pragma unroll
        for (int i = 0; i < kFinBatch; i++)
            if (s0 + i * kFinWaves < S) a += v[i];
    }
    part[wave][lane] = a;
    __syncthreads();
    if (wave == 0 && r < R) {
        float t = part[0][lane];
        #pragma unroll
        for (int w = 1; w < kFinWaves; w++) t += part[w][lane];
        y[b * R + r] = bf16_rne(t * scale);
    }
}


// Uncompressed FP8 GEMV, B = 1, for rows of more than 8192 columns (the
// baseline of the fused one there; shorter rows take gemm_raw_xs_kernel): a
// wave takes 4 rows; each lane walks 16-column blocks, so a wave's load is
// 1 KiB of one row, converting W to bf16 pairs and accumulating
// v_dot2_f32_bf16 against x read from global memory (cache-resident), then
// the wave sums its lanes.  C % 16 == 0.  At one batch row its whole-row
// loads stream W faster than gemm_raw_kernel (17 against 22 us for
// 17408 x 5120); from two rows on gemm_raw_kernel is faster.
constexpr int kRawRows = 4;

__device__ __forceinline__ float wave_sum(float v) {
    #pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// KS waves of a workgroup (of 4) take the same rows, each a contiguous
// range of column blocks, and add their sums in wave order through LDS: a
// matrix of few, long rows (5120 x 17408) then still runs enough waves.
template <int NB, int KS>
__global__ __launch_bounds__(256) void gemm_raw_dot2_kernel(const v4u* __restrict__ W, int64_t R,
                                                       int64_t C, const v4u* __restrict__ x,
                                                       float scale, uint16_t* __restrict__ y) {
    static_assert(KS == 1 || KS == 2 || KS == 4, "a workgroup is 4 waves");
    __shared__ float part[256 / kLanes][kRawRows][NB];
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = threadIdx.x / kLanes;
    const int ks = wave % KS;
    const int64_t r0 = ((int64_t)blockIdx.x * (256 / kLanes / KS) + wave / KS) * kRawRows;
    const int64_t cb = C / 16;                 // 16-column blocks per row
    const int64_t kb = (cb + KS - 1) / KS;     // of them per wave
    const int64_t k_end = std::min<int64_t>((int64_t)(ks + 1) * kb, cb);
    float acc[kRawRows][NB];
    #pragma unroll
    for (int i = 0; i < kRawRows; i++)
        #pragma unroll
        for (int b = 0; b < NB; b++) acc[i][b] = 0.0f;
    for (int64_t k = (int64_t)ks * kb + lane; k < k_end && r0 < R; k += kLanes) {
        v2bf wb[kRawRows][8];
        #pragma unroll
        for (int i = 0; i < kRawRows; i++) {
            const int64_t r = r0 + i < R ? r0 + i : R - 1;
            const v4u v = __builtin_nontemporal_load(W + r * cb + k);
            const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
            #pragma unroll
            for (int j = 0; j < 4; j++) {
                wb[i][2 * j] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wv[j], 1.0f, false);
                wb[i][2 * j + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wv[j], 1.0f, true);
            }
        }
        #pragma unroll
        for (int b = 0; b < NB; b++) {
            const v4u x0 = x[(b * C) / 8 + 2 * k];
            const v4u x1 = x[(b * C) / 8 + 2 * k + 1];
            const uint32_t xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            #pragma unroll
            for (int i = 0; i < kRawRows; i++)
                #pragma unroll
                for (int m = 0; m < 8; m++)
                    acc[i][b] = __builtin_amdgcn_fdot2_f32_bf16(
                        wb[i][m], __builtin_bit_cast(v2bf, xv[m]), acc[i][b], false);
        }
    }
    #pragma unroll
    for (int i = 0; i < kRawRows; i++)
        #pragma unroll
        for (int b = 0; b < NB; b++) {
            const float v = wave_sum(acc[i][b]);
            if (KS == 1) {
                if (lane == 0 && r0 + i < R) y[b * R + r0 + i] = bf16_rne(v * scale);
            } else if (lane == 0) {
                part[wave][i][b] = v;
            }
        }
    if constexpr (KS > 1) {
        __syncthreads();
        if (ks == 0 && lane < kRawRows * NB) {
            const int i = lane / NB, b = lane % NB;
            if (r0 + i < R) {
                float t = part[wave][i][b];
                #pragma unroll
                for (int q = 1; q < KS; q++) t += part[wave + q][i][b];
                y[b * R + r0 + i] = bf16_rne(t * scale);
            }
        }
    }
}

// Uncompressed FP8 skinny GEMM (the baseline of the fused one) on
// v_mfma_f32_4x4x4_16b_bf16, whose 16 independent 4x4x4 blocks let one load
// instruction cover 4 rows x 256 contiguous bytes.  Lane l = 4b + i holds
// row i of a row group: of each 256-column chunk, columns 16b .. 16b + 15
// (block b, four k-steps of 4 columns).  Lane 4b + j holds x[j] at the same
// columns (and x[j + 4] for a second product when B > 4), loaded once per
// chunk and used for all kRawGroups row groups of the wave; lanes j >= B
// load zeros.  Block b's 4 x 4 sums cover its own columns and sit in lane
// 4b + j, register i (row i, batch j).  A workgroup's waves take 4 *
// kRawGroups rows and split the chunks in contiguous ranges; at the end the
// 16 blocks are added by lane shuffles and the waves in wave order through
// LDS, so results are deterministic.  C % 16 == 0; y's batch rows are ldy
// apart (the launcher splits tall matrices into several launches).
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
constexpr int kRawMaxWaves = 8;      // waves per workgroup (up to 256 VGPRs each)
constexpr int kRawGroups = 5;        // row groups of 4 rows per wave: 20 rows a workgroup
constexpr int kRawChunk = 256;       // columns per chunk

// 4 bf16 from 4 FP8 bytes (exact).
__device__ __forceinline__ v4bf fp8x4_to_bf16(uint32_t w) {
    const v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    const v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    return v4bf{p0[0], p0[1], p1[0], p1[1]};
}

template <bool HI>   // HI: B > 4, a second product for batch rows 4..7
struct RawChunk {
    v4u w[kRawGroups];   // 16 FP8 of each row group
    v4u x[HI ? 4 : 2];   // 16 bf16 of x[j] (and x[j + 4])
};

template <bool HI>
__global__ __launch_bounds__(kRawMaxWaves * kLanes) void gemm_raw_kernel(
    const uint8_t* __restrict__ W, int64_t R, int64_t C, const uint16_t* __restrict__ x, int NB,
    float scale, uint16_t* __restrict__ y, int64_t ldy, int chunks_per_wave) {
    constexpr int NP = HI ? 2 : 1;
    __shared__ float part[kRawMaxWaves][kRawGroups][NP][16];
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = threadIdx.x / kLanes;
    const int nw = blockDim.x / kLanes;
    const int b = lane >> 2, i = lane & 3;       // block; row (A) or batch row (x)
    const int64_t row0 = (int64_t)blockIdx.x * (4 * kRawGroups);
    const int64_t n_chunks = (C + kRawChunk - 1) / kRawChunk;
    const int64_t c_begin = (int64_t)wave * chunks_per_wave;
    const int64_t c_end = c_begin + chunks_per_wave < n_chunks ? c_begin + chunks_per_wave : n_chunks;
    // Loads go through buffer resources (the launcher keeps R * C and B * C * 2
    // below 2^31 bytes): a lane out of range reads at kNoSeg, past the bound,
    // and gets zeros, so no load sits behind a branch and the wait counts stay
    // exact across the two chunks in flight.
    const Rsrc wsrc = rsrc(W, (uint32_t)(R * C));
    const Rsrc xsrc = rsrc(x, (uint32_t)(NB * C * 2));
    uint32_t woff[kRawGroups];
    #pragma unroll
    for (int g = 0; g < kRawGroups; g++) {
        const int64_t r = row0 + 4 * g + i;
        woff[g] = (uint32_t)((r < R ? r : R - 1) * C + 16 * b);   // rows past R repeat the last one
    }
    const uint32_t xoff0 = (uint32_t)(((int64_t)i * C + 16 * b) * 2);
    const uint32_t xoff1 = (uint32_t)(((int64_t)(i + 4) * C + 16 * b) * 2);
    const bool x0_in = i < NB, x1_in = i + 4 < NB;
    auto load = [&](int64_t c, RawChunk<HI>& k) {
        const int64_t col = c * kRawChunk;
        // C % 16 == 0: a lane's 16 columns are all in or all out
        const bool in = c < c_end && col + 16 * b < C;
        #pragma unroll
        for (int g = 0; g < kRawGroups; g++)
            k.w[g] = __builtin_amdgcn_raw_buffer_load_b128(
                wsrc, in ? woff[g] + (uint32_t)col : kNoSeg, 0, kNT);
        const uint32_t o0 = in && x0_in ? xoff0 + (uint32_t)col * 2u : kNoSeg;
        k.x[0] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, o0, 0, 0);
        k.x[1] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, o0, 16, 0);
        if constexpr (HI) {
            const uint32_t o1 = in && x1_in ? xoff1 + (uint32_t)col * 2u : kNoSeg;
            k.x[2] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, o1, 0, 0);
            k.x[3] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, o1, 16, 0);
        }
    };
    v4f acc[kRawGroups][NP];
    #pragma unroll
    for (int g = 0; g < kRawGroups; g++)
        #pragma unroll
        for (int p = 0; p < NP; p++) acc[g][p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma = [&](const RawChunk<HI>& k) {
        #pragma unroll
        for (int s = 0; s < 4; s++) {   // k-step: columns 16b + 4s .. + 3
            const uint32_t xs[4] = {k.x[0].x, k.x[0].y, k.x[0].z, k.x[0].w};
            const uint32_t xt[4] = {k.x[1].x, k.x[1].y, k.x[1].z, k.x[1].w};
            const v2u x0 = s < 2 ? v2u{xs[2 * s], xs[2 * s + 1]} : v2u{xt[2 * s - 4], xt[2 * s - 3]};
            v2u x1 = x0;
            if constexpr (HI) {
                const uint32_t xu[4] = {k.x[2].x, k.x[2].y, k.x[2].z, k.x[2].w};
                const uint32_t xv[4] = {k.x[3].x, k.x[3].y, k.x[3].z, k.x[3].w};
                x1 = s < 2 ? v2u{xu[2 * s], xu[2 * s + 1]} : v2u{xv[2 * s - 4], xv[2 * s - 3]};
            }
            #pragma unroll
            for (int g = 0; g < kRawGroups; g++) {
                const uint32_t ws[4] = {k.w[g].x, k.w[g].y, k.w[g].z, k.w[g].w};
                const v4bf a = fp8x4_to_bf16(ws[s]);
                acc[g][0] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
                    a, __builtin_bit_cast(v4bf, x0), acc[g][0], 0, 0, 0);
                if constexpr (HI)
                    acc[g][NP - 1] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
                        a, __builtin_bit_cast(v4bf, x1), acc[g][NP - 1], 0, 0, 0);
            }
        }
    };
    // two chunks in flight: one loads while the other multiplies (two
    // buffers in turn, so no register copy waits on a pending load); chunks
    // past c_end read zeros for W and x and add exact zeros
    RawChunk<HI> k0, k1;
    load(c_begin, k0);
    for (int64_t c = c_begin; c < c_end; c += 2) {
        load(c + 1, k1);
        mma(k0);
        load(c + 2, k0);
        mma(k1);
    }
    // add the 16 blocks: lanes with equal lane mod 4 (every lane gets the sum)
    #pragma unroll
    for (int g = 0; g < kRawGroups; g++)
        #pragma unroll
        for (int p = 0; p < NP; p++)
            #pragma unroll
            for (int m = 4; m < kLanes; m <<= 1)
                #pragma unroll
                for (int v = 0; v < 4; v++) acc[g][p][v] += __shfl_xor(acc[g][p][v], m, kLanes);
    if (lane < 4) {   // lane j: batch row j (and j + 4), register v: row v of the group
        #pragma unroll
        for (int g = 0; g < kRawGroups; g++)
            #pragma unroll
            for (int p = 0; p < NP; p++)
                #pragma unroll
                for (int v = 0; v < 4; v++) part[wave][g][p][4 * v + lane] = acc[g][p][v];
    }
    __syncthreads();
    // 16 * kRawGroups * NP outputs (more than the threads of a one-wave
    // workgroup when B > 4): each the waves' sums in wave order
    for (int t = threadIdx.x; t < 16 * kRawGroups * NP; t += blockDim.x) {
        const int g = t / (16 * NP), p = (t / 16) % NP, v = (t / 4) % 4, j = t % 4;
        const int64_t row = row0 + 4 * g + v;
        const int bn = j + 4 * p;
        if (row >= R || bn >= NB) continue;
        float sum = part[0][g][p][4 * v + j];
        for (int w = 1; w < nw; w++) sum += part[w][g][p][4 * v + j];
        y[(int64_t)bn * ldy + row] = bf16_rne(sum * scale);
    }
}

// The same products with x held in registers (rows of at most kXsMaxChunks
// chunks: 8192 columns; every B, lanes j >= B hold zeros).  Lanes, blocks
// and chunks as in gemm_raw_kernel.
// Each wave owns CPW consecutive chunks and loads x for them once, before
// its loop; it then streams the workgroup's row groups over its chunks,
// PIPE row groups of loads in flight in PIPE buffers taken in turn.  So the
// loop issues only W loads, and its waits cover only them.  A row group's
// 16 blocks are added by two DPP rotations inside each 16-lane row and
// three v_permlane16/32_swap across rows; lanes 16v + j store the wave's
// sum of row v for batch row j to LDS, and the workgroup adds them at the
// end in wave order, so results are deterministic.  Out-of-range rows and chunks read zeros
// through the buffer bound: a lane's offset past the workgroup's last row
// or its matrix row stays past the bound for every row group it adds.
constexpr int kXsMaxWaves = 16;
constexpr int kXsMaxRg = 32;      // row groups of 4 rows per workgroup
constexpr int kXsMaxChunks = 32;  // chunks of 256 columns per row (16 waves of 2)

// v_permlane16_swap (H32 false) or v_permlane32_swap of a and c, and the sum
// of the two registers it leaves: rows of 16 lanes (a0 + a1, c0 + c1,
// a2 + a3, c2 + c3), or halves of 32 (a_lo + a_hi, c_lo + c_hi).  The
// builtin's result is read through a 64-bit bit cast: indexing its vector
// type reads the first element twice with this compiler.
template <bool H32>
__device__ __forceinline__ float swap_add(float a, float c) {
    const uint32_t ua = __builtin_bit_cast(uint32_t, a), uc = __builtin_bit_cast(uint32_t, c);
    uint64_t u;
    if constexpr (H32) u = __builtin_bit_cast(uint64_t, __builtin_amdgcn_permlane32_swap(ua, uc, false, false));
    else u = __builtin_bit_cast(uint64_t, __builtin_amdgcn_permlane16_swap(ua, uc, false, false));
    return __builtin_bit_cast(float, (uint32_t)u) + __builtin_bit_cast(float, (uint32_t)(u >> 32));
}

template <bool HI, int CPW, int PIPE>
__global__ __launch_bounds__(kXsMaxWaves * kLanes) void gemm_raw_xs_kernel(
    const uint8_t* __restrict__ W, int64_t R, int64_t C, const uint16_t* __restrict__ x, int NB,
    float scale, uint16_t* __restrict__ y, int64_t ldy, int rg_per_block) {
    constexpr int NP = HI ? 2 : 1;
    __shared__ float part[kXsMaxWaves][kXsMaxRg][NP][4][4];   // [.][.][.][batch j][row v]
    const int lane = threadIdx.x & (kLanes - 1);
    const int wave = threadIdx.x / kLanes;
    const int nw = blockDim.x / kLanes;
    const int b = lane >> 2, i = lane & 3;
    const int64_t rg0 = (int64_t)blockIdx.x * rg_per_block;
    const int64_t n_rg_all = (R + 3) / 4;
    const int n_rg = (int)(n_rg_all - rg0 < rg_per_block ? n_rg_all - rg0 : rg_per_block);
    const int64_t row_end = 4 * (rg0 + n_rg) < R ? 4 * (rg0 + n_rg) : R;
    const int64_t n_chunks = (C + kRawChunk - 1) / kRawChunk;
    // the launcher keeps R * C below 2^31 and every offset a workgroup forms,
    // the row groups it loads past its end included, below 2^32
    const uint32_t bound = (uint32_t)(row_end * C);
    const Rsrc wsrc = rsrc(W, bound);
    const Rsrc xsrc = rsrc(x, (uint32_t)(NB * C * 2));
    v4u xr[CPW][NP][2];   // x[i] (and x[i + 4]) at columns 16b .. 16b + 15 of each chunk
    uint32_t woff[CPW];   // row i of row group 0, the lane's 16 columns of each chunk
    #pragma unroll
    for (int j = 0; j < CPW; j++) {
        const int64_t ch = (int64_t)wave * CPW + j;
        const int64_t col = ch * kRawChunk + 16 * b;
        const bool in = ch < n_chunks && col < C;   // C % 16 == 0
        woff[j] = in ? (uint32_t)((4 * rg0 + i) * C + col) : bound;
        #pragma unroll
        for (int p = 0; p < NP; p++) {
            const uint32_t o = in && i + 4 * p < NB ? (uint32_t)(((i + 4 * p) * C + col) * 2) : kNoSeg;
            xr[j][p][0] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, o, 0, 0);
            xr[j][p][1] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, o, 16, 0);
        }
    }
    // Issue order is what the waits count: the x loads, then the row groups
    // in order.  The loop's wait for row group s then covers x and leaves
    // the later row groups in flight; without the barriers the compiler
    // moves loads past each other and the first wait is for all of them.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t rg_bytes = (uint32_t)(4 * C);
    v4u wb[PIPE][CPW];
    auto load = [&](int s, v4u (&buf)[CPW]) {   // row group s of the workgroup
        #pragma unroll
        for (int j = 0; j < CPW; j++)
            buf[j] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, woff[j] + (uint32_t)s * rg_bytes,
                                                           0, kNT);
    };
    #pragma unroll
    for (int p = 0; p < PIPE; p++) {
        load(p, wb[p]);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
    // every workgroup has a row group (the launcher sizes the grid so), and
    // a loop with no zero-trip test keeps the loads above where they are
    const int n_iter = (n_rg + PIPE - 1) / PIPE;
    int it = 0;
    do {
        static_for<0, PIPE>([&](auto P) {
            constexpr int q = decltype(P)::value;
            const int s = it * PIPE + q;
            v4f acc[NP];
            #pragma unroll
            for (int p = 0; p < NP; p++) acc[p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            // the row group's W as bf16 first, so that its buffer takes the
            // load of row group s + PIPE before the products (17408 x 5120 at
            // B = 8: 18.5 -> 17.8 us per call)
            v4bf a[CPW][4];
            #pragma unroll
            for (int j = 0; j < CPW; j++) {
                const uint32_t ws[4] = {wb[q][j].x, wb[q][j].y, wb[q][j].z, wb[q][j].w};
                #pragma unroll
                for (int k = 0; k < 4; k++) a[j][k] = fp8x4_to_bf16(ws[k]);
            }
            load(s + PIPE, wb[q]);
            #pragma unroll
            for (int j = 0; j < CPW; j++) {
                #pragma unroll
                for (int k = 0; k < 4; k++) {   // k-step: columns 16b + 4k .. + 3
                    #pragma unroll
                    for (int p = 0; p < NP; p++) {
                        const v4u& xv = xr[j][p][k >> 1];
                        const v2u xk = (k & 1) ? v2u{xv.z, xv.w} : v2u{xv.x, xv.y};
                        acc[p] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
                            a[j][k], __builtin_bit_cast(v4bf, xk), acc[p], 0, 0, 0);
                    }
                }
            }
            #pragma unroll
            for (int p = 0; p < NP; p++) {
                float t[4];
                // blocks 4r .. 4r + 3 of each 16-lane row r (DPP row_ror 4, 8)
                #pragma unroll
                for (int v = 0; v < 4; v++) {
                    t[v] = acc[p][v];
                    t[v] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                        0, __builtin_bit_cast(int, t[v]), 0x124, 0xF, 0xF, false));
                    t[v] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                        0, __builtin_bit_cast(int, t[v]), 0x128, 0xF, 0xF, false));
                }
                // then the rows: register v's rows 0 + 1 and 2 + 3 paired with
                // register v + 1's, then the halves, so that row v of the
                // result holds register v's total (lanes 16v + j: batch row j)
                const float tot = swap_add<true>(swap_add<false>(t[0], t[1]),
                                                 swap_add<false>(t[2], t[3]));
                if (s < n_rg && (lane & 15) < 4) part[wave][s][p][lane & 3][lane >> 4] = tot;
            }
        });
    } while (++it < n_iter);
    __syncthreads();
    // outputs (row r of the workgroup, batch row bn), rows consecutive per thread
    const int rows = (int)(row_end - 4 * rg0);
    for (int t = threadIdx.x; t < rows * NB; t += blockDim.x) {
        const int bn = t / rows, r = t % rows;
        const int s = r / 4, v = r % 4, p = bn / 4, j = bn % 4;
        float sum = part[0][s][p][j][v];
        for (int w = 1; w < nw; w++) sum += part[w][s][p][j][v];
        y[(int64_t)bn * ldy + 4 * rg0 + r] = bf16_rne(sum * scale);
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

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// A launch's work-item count per grid dimension is a 32-bit number.
bool grid_fits(int64_t blocks, int64_t threads) {
    return blocks >= 0 && blocks <= int64_t(UINT32_MAX) / threads;
}

// The streaming kernels take one 16-byte vector per thread, so one launch
// covers at most 2^31 vectors (32 GiB per tensor); larger tensors go in
// several launches on the same stream.
constexpr int64_t kMaxLaunchVecs = int64_t(1) << 31;

// Compute units of the current device, queried once per device.
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < kMaxDevices) {
        const int known = g_cu_count[dev].load(std::memory_order_relaxed);
        if (known > 0) return known;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (dev < kMaxDevices && cus > 0) g_cu_count[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

int sps_for(int32_t log2L) {
    return log2L == TANS_PAIR_LOG2L ? 2 : (log2L == TANS_NIBBLE_LOG2L ? 1 : 0);
}

template <int SPS>
constexpr int kFusedGroups = 1;   // groups per wave in the fused kernel

int gemm_fused_launch(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                      const uint16_t* states, const void* sm, const uint32_t* table,
                      int32_t log2L, int64_t R, int64_t C, int64_t S, int64_t Nc, const void* x,
                      int64_t B, float scale, void* workspace, int64_t workspace_bytes, void* y,
                      void* stream);

// Device scratch of tans_fp8_gemm_fused_noalloc: the per-segment partial
// sums live in this file-scope array, so that entry point allocates
// nothing.  Each GPU holds its own copy for the life of the process.  In
// host code `scratch` is only a handle: its device address on the current
// GPU comes from hipGetSymbolAddress, looked up once per device and kept.
constexpr int64_t kGemmScratchBytes = int64_t(16) << 20;
static __device__ __align__(256) float scratch[kGemmScratchBytes / 4];

std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices];

int scratch_address(void** out) {
    int dev = -1;
    int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc != TANS_OK) return rc;
    if (dev < 0 || dev >= kMaxDevices) return fail(TANS_EINVAL, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                       "hipGetSymbolAddress(scratch)");
        if (rc != TANS_OK) return rc;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return TANS_OK;
}

}  // namespace

extern "C" {

int tans_fp8_memcpy(const void* a, void* c, int64_t n, void* stream) {
    if (n < 0 || n % 16 || ((!a || !c) && n)) return fail(TANS_EINVAL, "memcpy: n must be a multiple of 16");
    if (n == 0) return TANS_OK;
    if (!aligned(a, 16) || !aligned(c, 16)) return fail(TANS_EINVAL, "memcpy: buffers must be 16-byte aligned");
    const int64_t n_vec = n / 16;
    for (int64_t v0 = 0; v0 < n_vec; v0 += kMaxLaunchVecs) {
        const int64_t m = std::min(kMaxLaunchVecs, n_vec - v0);
        hipLaunchKernelGGL(fp8_copy_kernel, dim3((unsigned)((m + kBlock - 1) / kBlock)), dim3(kBlock),
                           0, (hipStream_t)stream, (const v4u*)a + v0, (v4u*)c + v0, m);
        const int rc = hip_check(hipGetLastError(), "fp8_copy_kernel launch");
        if (rc != TANS_OK) return rc;
    }
    return TANS_OK;
}

int tans_fp8_vecadd_raw(const void* a, const void* b, void* c, int64_t n, void* stream) {
    if (n < 0 || n % 16 || ((!a || !b || !c) && n)) return fail(TANS_EINVAL, "vecadd_raw: n must be a multiple of 16");
    if (n == 0) return TANS_OK;
    if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16))
        return fail(TANS_EINVAL, "vecadd_raw: buffers must be 16-byte aligned");
    const int64_t n_vec = n / 16;
    for (int64_t v0 = 0; v0 < n_vec; v0 += kMaxLaunchVecs) {
        const int64_t m = std::min(kMaxLaunchVecs, n_vec - v0);
        hipLaunchKernelGGL(fp8_add_kernel, dim3((unsigned)((m + kBlock - 1) / kBlock)), dim3(kBlock),
                           0, (hipStream_t)stream, (const v4u*)a + v0, (const v4u*)b + v0,
                           (v4u*)c + v0, m);
        const int rc = hip_check(hipGetLastError(), "fp8_add_kernel launch");
        if (rc != TANS_OK) return rc;
    }
    return TANS_OK;
}

int tans_stream_probe(int32_t mode, int32_t nontemporal, const void* a, const void* b, void* c,
                      int64_t n, void* sink, void* stream) {
    if (mode < 0 || mode > 2) return fail(TANS_EINVAL, "stream_probe: mode must be 0, 1 or 2");
    if (n < 0 || n % 16) return fail(TANS_EINVAL, "stream_probe: n must be a multiple of 16");
    if (n == 0) return TANS_OK;
    const bool need_a = mode != 1, need_b = mode == 2, need_c = mode != 0;
    if ((need_a && !a) || (need_b && !b) || (need_c && !c) || (mode == 0 && !sink))
        return fail(TANS_EINVAL, "stream_probe: null pointer");
    if ((need_a && !aligned(a, 16)) || (need_b && !aligned(b, 16)) || (need_c && !aligned(c, 16)) ||
        (mode == 0 && !aligned(sink, 4)))
        return fail(TANS_EINVAL, "stream_probe: buffers must be 16-byte aligned");
    const int64_t n_vec = n / 16;
    for (int64_t v0 = 0; v0 < n_vec; v0 += kMaxLaunchVecs) {
        const int64_t m = std::min(kMaxLaunchVecs, n_vec - v0);
        const dim3 grid((unsigned)((m + kBlock - 1) / kBlock));
        const v4u* pa = need_a ? (const v4u*)a + v0 : nullptr;
        const v4u* pb = need_b ? (const v4u*)b + v0 : nullptr;
        v4u* pc = need_c ? (v4u*)c + v0 : nullptr;
        auto launch = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(kBlock), 0, (hipStream_t)stream, pa, pb, pc, m,
                               (uint32_t*)sink);
        };
        switch (mode * 2 + (nontemporal ? 1 : 0)) {
            case 0: launch(stream_probe_kernel<0, false>); break;
            case 1: launch(stream_probe_kernel<0, true>); break;
            case 2: launch(stream_probe_kernel<1, false>); break;
            case 3: launch(stream_probe_kernel<1, true>); break;
            case 4: launch(stream_probe_kernel<2, false>); break;
            default: launch(stream_probe_kernel<2, true>); break;
        }
        const int rc = hip_check(hipGetLastError(), "stream_probe_kernel launch");
        if (rc != TANS_OK) return rc;
    }
    return TANS_OK;
}

int tans_build_decode_table_device(const int32_t* spread, const int32_t* freqs, int32_t nsym,
                                   int32_t log2L, uint32_t* table, int32_t* status,
                                   void* stream) {
    if (!spread || !freqs || !table) return fail(TANS_EINVAL, "table: null pointer");
    if (!((nsym == 256 && log2L == TANS_PAIR_LOG2L) || (nsym == 16 && log2L == TANS_NIBBLE_LOG2L)))
        return fail(TANS_EINVAL, "table: need (nsym 256, log2L 12) or (nsym 16, log2L 11)");
    if (status && !aligned(status, 4)) return fail(TANS_EINVAL, "table: status must be 4-byte aligned");
    hipLaunchKernelGGL(table_kernel, dim3(1), dim3(kTableWaves * 64), 0, (hipStream_t)stream, spread, freqs,
                       (int)nsym, (int)log2L, (v2u*)table, status);
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
    if (!a_comp || !a_offsets || !a_sm || !b_comp || !b_offsets || !b_sm || !table || !out)
        return fail(TANS_EINVAL, "vecadd_fused: null pointer");
    // no state arrays: the packed layout of short streams
    const bool packed = !a_states;
    if (packed != !b_states)
        return fail(TANS_EINVAL, "vecadd_fused: A and B must both have states or both be packed");
    if (packed && (sps != 2 || N > 16 * kPackMaxSegs))
        return fail(TANS_EINVAL, "vecadd_fused: the packed layout needs the pair table (log2L 12) "
                                 "and N <= 64");
    if (a_comp_bytes < 0 || b_comp_bytes < 0 || a_comp_bytes % 4 || b_comp_bytes % 4)
        return fail(TANS_EINVAL, "vecadd_fused: compressed sizes must be multiples of 4 bytes");
    if (!aligned(a_comp, 16) || !aligned(b_comp, 16) || !aligned(a_sm, 8) || !aligned(b_sm, 8) ||
        !aligned(a_offsets, 8) || !aligned(b_offsets, 8) || !aligned(a_states, 2) ||
        !aligned(b_states, 2) || !aligned(table, 8) || !aligned(out, 16))
        return fail(TANS_EINVAL, "vecadd_fused: misaligned buffer (comp and out 16, sm 8 bytes)");
    if (N / kTile > INT32_MAX) return fail(TANS_EINVAL, "vecadd_fused: N too large");
    const int64_t groups = (K + kLanes - 1) / kLanes;
    const int64_t per_block = (int64_t)kDecWaves * (sps == 2 ? kFusedGroups<2> : kFusedGroups<1>);
    // one workgroup per CU at most; the waves loop over the groups
    const int cus = cu_count();
    if (cus <= 0) return fail(TANS_EHIP, "vecadd_fused: cannot query the device's CU count");
    const int64_t blocks = std::min<int64_t>((groups + per_block - 1) / per_block, cus);
    const int n_tiles = (int)(N / kTile);
#define TANS_LAUNCH_FUSED(S, FIRST)                                                               \
    hipLaunchKernelGGL((fused_add_kernel<S, kFusedGroups<S>, FIRST>), dim3((unsigned)blocks),       \
                       dim3(kDecBlock), 0, (hipStream_t)stream, (const uint32_t*)a_comp,         \
                       a_comp_bytes / 4, a_offsets, a_states, (const v2u*)a_sm,                  \
                       (const uint32_t*)b_comp, b_comp_bytes / 4, b_offsets, b_states,           \
                       (const v2u*)b_sm, (const v2u*)table, K, n_tiles, (v4u*)out)
    // streams that fit the ring are loaded whole at their start
    if (packed) {
        switch (n_tiles) {
            case 1: TANS_LAUNCH_FUSED(2, -1); break;
            case 2: TANS_LAUNCH_FUSED(2, -2); break;
            case 3: TANS_LAUNCH_FUSED(2, -3); break;
            default: TANS_LAUNCH_FUSED(2, -4); break;
        }
    } else if (sps == 2) {
        if (n_tiles == 1) TANS_LAUNCH_FUSED(2, Alpha<2>::kOneTileSegs);
        else if (n_tiles <= Alpha<2>::kResidentTiles) TANS_LAUNCH_FUSED(2, kSlots);
        else TANS_LAUNCH_FUSED(2, 0);
    } else {
        if (n_tiles == 1) TANS_LAUNCH_FUSED(1, Alpha<1>::kOneTileSegs);
        else if (n_tiles <= Alpha<1>::kResidentTiles) TANS_LAUNCH_FUSED(1, kSlots);
        else TANS_LAUNCH_FUSED(1, 0);
    }
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
    if (!comp || !offsets || !sm || !table || !out)
        return fail(TANS_EINVAL, "decode: null pointer");
    // no state array: the packed layout of short streams
    const bool packed = !states;
    if (packed && (sps != 2 || N > 16 * kPackMaxSegs))
        return fail(TANS_EINVAL, "decode: the packed layout needs the pair table (log2L 12) and "
                                 "N <= 64");
    if (comp_bytes < 0 || comp_bytes % 4)
        return fail(TANS_EINVAL, "decode: compressed size must be a multiple of 4 bytes");
    if (!aligned(comp, 16) || !aligned(sm, 8) || !aligned(offsets, 8) || !aligned(states, 2) ||
        !aligned(table, 8) || !aligned(out, 4))
        return fail(TANS_EINVAL, "decode: misaligned buffer (comp 16, sm 8, out 4 bytes)");
    if ((N + kTile - 1) / kTile > INT32_MAX) return fail(TANS_EINVAL, "decode: N too large");
    // the stores address 4 rows of a tile with 32-bit offsets
    if (K > (int64_t(1) << 30)) return fail(TANS_EINVAL, "decode: more than 2^30 lanes");
    const int64_t groups = (K + kLanes - 1) / kLanes;
    const int64_t per_block = (int64_t)kDecWaves * kDecodeGroups;
    int64_t blocks = (groups + per_block - 1) / per_block;
    // Columns of one or two tiles: one workgroup per CU, the waves loop over
    // their group pairs (measured at 2^30 elements: 16 per column 923 ->
    // 616 us).  From 4 tiles on, one workgroup per 32 groups is as fast or
    // faster (64 per column: 472 vs 468 us; 256: 388 vs 400 us).
    if ((N + kTile - 1) / kTile <= 2) {
        const int cus = cu_count();
        if (cus <= 0) return fail(TANS_EHIP, "decode: cannot query the device's CU count");
        blocks = std::min<int64_t>(blocks, cus);
    }
    if (!grid_fits(blocks, kDecBlock)) return fail(TANS_EINVAL, "decode: K too large");
#define TANS_LAUNCH_DECODE(S, FIRST)                                                              \
    hipLaunchKernelGGL((decode_kernel<S, FIRST>), dim3((unsigned)blocks),                        \
                       dim3(kDecBlock), 0, (hipStream_t)stream, (const uint32_t*)comp,           \
                       comp_bytes / 4, offsets, states, (const v2u*)sm, (const v2u*)table, K, N, \
                       (uint8_t*)out)
    // streams that fit the ring are loaded whole at their start
    const int64_t n_tiles = (N + kTile - 1) / kTile;
    if (packed) {
        switch (n_tiles) {
            case 1: TANS_LAUNCH_DECODE(2, -1); break;
            case 2: TANS_LAUNCH_DECODE(2, -2); break;
            case 3: TANS_LAUNCH_DECODE(2, -3); break;
            default: TANS_LAUNCH_DECODE(2, -4); break;
        }
    } else if (sps == 2) {
        if (n_tiles == 1) TANS_LAUNCH_DECODE(2, Alpha<2>::kOneTileSegs);
        else if (n_tiles <= Alpha<2>::kResidentTiles) TANS_LAUNCH_DECODE(2, kSlots);
        else TANS_LAUNCH_DECODE(2, 0);
    } else {   // (the nibble decoder loaded whole at two tiles spills registers)
        if (n_tiles == 1) TANS_LAUNCH_DECODE(1, Alpha<1>::kOneTileSegs);
        else TANS_LAUNCH_DECODE(1, 0);
    }
#undef TANS_LAUNCH_DECODE
    return hip_check(hipGetLastError(), "decode_kernel launch");
}

int tans_fp8_gemm_fused(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                        const uint16_t* states, const void* sm, const uint32_t* table,
                        int32_t log2L, int64_t R, int64_t C, int64_t S, int64_t Nc, const void* x,
                        int64_t B, float scale, void* workspace, int64_t workspace_bytes, void* y,
                        void* stream) {
    return gemm_fused_launch(comp, comp_bytes, offsets, states, sm, table, log2L, R, C, S, Nc, x,
                             B, scale, workspace, workspace_bytes, y, stream);
}

int tans_fp8_gemm_fused_noalloc(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                                const uint16_t* states, const void* sm, const uint32_t* table,
                                int32_t log2L, int64_t R, int64_t C, int64_t S, int64_t Nc,
                                const void* x, int64_t B, float scale, void* y, void* stream) {
    // S * B * Rp floats of partial sums must fit the scratch array
    // (compared by division, so no product can overflow)
    const int64_t cap = kGemmScratchBytes / 4;
    const int64_t Rp = R > 0 && R <= cap ? (R + kLanes - 1) / kLanes * kLanes : cap + 1;
    if (R > 0 && S > 0 && B > 0 && (Rp > cap || S > cap / Rp || B > cap / (S * Rp)))
        return fail(TANS_EINVAL, "gemm_fused_noalloc: S * B * Rp * 4 bytes of partial sums "
                                 "exceed the 16 MiB device scratch buffer");
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc != TANS_OK) return rc;
    return gemm_fused_launch(comp, comp_bytes, offsets, states, sm, table, log2L, R, C, S, Nc, x,
                             B, scale, ws, kGemmScratchBytes, y, stream);
}

}  // extern "C"

namespace {

int gemm_fused_launch(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                      const uint16_t* states, const void* sm, const uint32_t* table,
                      int32_t log2L, int64_t R, int64_t C, int64_t S, int64_t Nc, const void* x,
                      int64_t B, float scale, void* workspace, int64_t workspace_bytes, void* y,
                      void* stream) {
    const int sps = sps_for(log2L);
    if (!sps) return fail(TANS_EINVAL, "gemm_fused: log2L must be 12 (pair) or 11 (nibble)");
    if (R <= 0 || C <= 0 || S <= 0 || Nc <= 0 || Nc % 32)
        return fail(TANS_EINVAL, "gemm_fused: need R, C, S > 0 and a segment width divisible by 32");
    if (Nc > kGemmMaxSegCols) return fail(TANS_EINVAL, "gemm_fused: segment width above 1024");
    if (S * Nc < C || (S - 1) * Nc >= C)
        return fail(TANS_EINVAL, "gemm_fused: S segments of Nc columns must cover C exactly");
    if (B < 1 || B > kGemmMaxBatch) return fail(TANS_EINVAL, "gemm_fused: batch must be 1..8");
    if (!comp || !offsets || !states || !sm || !table || !x || !workspace || !y)
        return fail(TANS_EINVAL, "gemm_fused: null pointer");
    if (comp_bytes < 0 || comp_bytes % 4)
        return fail(TANS_EINVAL, "gemm_fused: compressed size must be a multiple of 4 bytes");
    if (!aligned(comp, 16) || !aligned(sm, 8) || !aligned(offsets, 8) || !aligned(states, 2) ||
        !aligned(table, 8) || !aligned(x, 2) || !aligned(workspace, 16) || !aligned(y, 2))
        return fail(TANS_EINVAL, "gemm_fused: misaligned buffer (comp and workspace 16, sm 8 bytes)");
    const int64_t Rp = (R + kLanes - 1) / kLanes * kLanes;
    if (workspace_bytes < S * B * Rp * 4)
        return fail(TANS_EINVAL, "gemm_fused: workspace smaller than S * B * Rp * 4 bytes");
    const int64_t n_rg = Rp / kGemmGroupRows;
    const int64_t row_blocks = (n_rg + kGemmGroupsPerBlock - 1) / kGemmGroupsPerBlock;
    const int64_t blocks = S * row_blocks;
    if (!grid_fits(blocks, kDecBlock) || !grid_fits(B * (Rp / kLanes), kFinWaves * kLanes))
        return fail(TANS_EINVAL, "gemm_fused: matrix too large");
    hipStream_t st = (hipStream_t)stream;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kDecBlock), 0, st,
                           (const uint32_t*)comp, comp_bytes / 4, offsets, states, (const v2u*)sm,
                           (const v2u*)table, Rp, C, (int)S, (int)Nc, (int)row_blocks,
                           (const uint16_t*)x, (int)B, (float*)workspace);
    };
    if (sps == 2) launch(gemm_fused_kernel<2>); else launch(gemm_fused_kernel<1>);
    int rc = hip_check(hipGetLastError(), "gemm_fused_kernel launch");
    if (rc != TANS_OK) return rc;
    hipLaunchKernelGGL(gemm_finalize_kernel, dim3((unsigned)(B * (Rp / kLanes))),
                       dim3(kFinWaves * kLanes), 0, st, (const float*)workspace, (int)S, (int)B, Rp,
                       R, scale, (uint16_t*)y);
    return hip_check(hipGetLastError(), "gemm_finalize_kernel launch");
}

}  // namespace

extern "C" {

int tans_fp8_gemm_raw(const void* w, int64_t R, int64_t C, const void* x, int64_t B, float scale,
                      void* y, void* stream) {
    if (R <= 0 || C <= 0 || C % 16) return fail(TANS_EINVAL, "gemm_raw: need R > 0 and C a positive multiple of 16");
    if (B < 1 || B > kGemmMaxBatch) return fail(TANS_EINVAL, "gemm_raw: batch must be 1..8");
    if (!w || !x || !y) return fail(TANS_EINVAL, "gemm_raw: null pointer");
    if (!aligned(w, 16) || !aligned(x, 16) || !aligned(y, 2))
        return fail(TANS_EINVAL, "gemm_raw: W and x must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int64_t n_chunks = (C + kRawChunk - 1) / kRawChunk;
    if (B == 1 && n_chunks > kXsMaxChunks) {
        // rows of more than 8192 columns: the row-streaming kernel, each row
        // split over 2 or 4 waves, about 2.5 KiB or more of it each
        // (5120 x 17408: 4 waves, 17.4 against 24.1 us per call on MI355X)
        const int ks = C >= 10240 ? 4 : 2;
        const int64_t rows_per_block = (256 / kLanes) / ks * kRawRows;
        const int64_t blocks = (R + rows_per_block - 1) / rows_per_block;
        if (!grid_fits(blocks, 256)) return fail(TANS_EINVAL, "gemm_raw: matrix too large");
        auto launch = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(256), 0, st, (const v4u*)w, R,
                               C, (const v4u*)x, scale, (uint16_t*)y);
        };
        if (ks == 2) launch(gemm_raw_dot2_kernel<1, 2>);
        else launch(gemm_raw_dot2_kernel<1, 4>);
        return hip_check(hipGetLastError(), "gemm_raw_dot2_kernel launch");
    }
    const int cus = cu_count();
    if (cus <= 0) return fail(TANS_EHIP, "gemm_raw: cannot query the device's CU count");
    if ((int64_t)B * C * 2 > INT32_MAX) return fail(TANS_EINVAL, "gemm_raw: rows too long");
    if (n_chunks <= kXsMaxChunks) {
        // x in registers: one chunk per wave up to 16 chunks, then two; row
        // groups split evenly over about one workgroup per CU.  Measured on
        // 17408 x 5120 (10 waves of 2 chunks) at B = 2 / 4 / 8: 15.7 / 16.3 /
        // 18.0 us per call, against 19.1 / 20.8 / 25.9 us with gemm_raw_kernel
        // (4 or 8 row groups in flight: 16.0-17.2 / 16.7-17.7 / 18.8-20.0 us);
        // at B = 1 15.6 us against 16.4 us with gemm_raw_dot2_kernel.  With
        // each row group's reload issued before its products: 15.5 / 15.8 /
        // 16.1 / 17.8 us at B = 1 / 2 / 4 / 8.
        // Longer rows stay with gemm_raw_kernel: on 5120 x 17408 a wave of
        // this kernel would hold 9 chunks of x and stream only 5 row groups; it
        // measured 18.8 / 19.9 / 23.6 against 18.4 / 19.3 / 24.0 us.
        const int cpw = n_chunks <= 16 ? 1 : 2;
        const int64_t nw = (n_chunks + cpw - 1) / cpw;
        const int pipe = cpw == 1 ? 8 : 6;
        const int64_t n_rg = (R + 3) / 4;
        const int64_t rgb = std::min<int64_t>(kXsMaxRg, (n_rg + cus - 1) / cus);
        // launches of at most rows_per_launch rows keep each W slice below
        // 2^31 bytes; the loads a workgroup issues past its last row reach
        // at most 4 * (rgb + 2 * pipe) + 4 rows further, so every offset
        // stays below 2^32
        const int64_t rows_per_launch =
            std::max<int64_t>(4 * rgb, INT32_MAX / C / (4 * rgb) * (4 * rgb));
        if ((4 * (rgb + 2 * pipe) + 4) * C > INT32_MAX)
            return fail(TANS_EINVAL, "gemm_raw: rows too long");
        for (int64_t r0 = 0; r0 < R; r0 += rows_per_launch) {
            const int64_t rl = std::min(rows_per_launch, R - r0);
            const int64_t blocks = ((rl + 3) / 4 + rgb - 1) / rgb;
            if (!grid_fits(blocks, kXsMaxWaves * kLanes))
                return fail(TANS_EINVAL, "gemm_raw: matrix too large");
            auto launch = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3((unsigned)(nw * kLanes)),
                                   0, st, (const uint8_t*)w + r0 * C, rl, C, (const uint16_t*)x,
                                   (int)B, scale, (uint16_t*)y + r0, R, (int)rgb);
            };
            if (B > 4) {
                if (cpw == 1) launch(gemm_raw_xs_kernel<true, 1, 8>);
                else launch(gemm_raw_xs_kernel<true, 2, 6>);
            } else {
                if (cpw == 1) launch(gemm_raw_xs_kernel<false, 1, 8>);
                else launch(gemm_raw_xs_kernel<false, 2, 6>);
            }
            const int rc = hip_check(hipGetLastError(), "gemm_raw_xs_kernel launch");
            if (rc != TANS_OK) return rc;
        }
        return TANS_OK;
    }
    // Workgroups of 4 * kRawGroups rows; their waves split the row's chunks
    // in contiguous ranges.  Up to one workgroup per CU (5120 rows: 256
    // workgroups of 20 rows on MI355X) takes 8 waves each; more workgroups
    // take 3, so that 4 or 5 of them share a CU and every one is resident
    // at once (17408 rows: 871 workgroups).  Measured on 5120 x 17408 at
    // B = 2 / 4 / 8: 17.8 / 19.2 / 24.0 us, against 24.8 / 27.8 / 36.2 us with
    // 16-row workgroups (320 of them, so 64 CUs held two); on 17408 x 5120:
    // 19.1 / 20.7 / 25.8 against 19.7 / 21.9 / 28.1 us.
    const int64_t rows_wg = 4 * kRawGroups;
    if (C > INT32_MAX / rows_wg)
        return fail(TANS_EINVAL, "gemm_raw: rows too long");
    // launches of at most rows_per_launch rows keep each W slice below 2^31 bytes
    const int64_t rows_per_launch = std::max<int64_t>(rows_wg, INT32_MAX / C / rows_wg * rows_wg);
    for (int64_t r0 = 0; r0 < R; r0 += rows_per_launch) {
        const int64_t rl = std::min(rows_per_launch, R - r0);
        const int64_t blocks = (rl + rows_wg - 1) / rows_wg;
        int64_t nw = blocks <= cus ? kRawMaxWaves : 3;
        nw = std::min<int64_t>(nw, n_chunks);
        const int64_t cpw = (n_chunks + nw - 1) / nw;        // chunks per wave
        nw = (n_chunks + cpw - 1) / cpw;                      // waves with chunks
        if (!grid_fits(blocks, kRawMaxWaves * kLanes))
            return fail(TANS_EINVAL, "gemm_raw: matrix too large");
        auto launch = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3((unsigned)(nw * kLanes)), 0,
                               st, (const uint8_t*)w + r0 * C, rl, C, (const uint16_t*)x, (int)B,
                               scale, (uint16_t*)y + r0, R, (int)cpw);
        };
        if (B > 4) launch(gemm_raw_kernel<true>); else launch(gemm_raw_kernel<false>);
        const int rc = hip_check(hipGetLastError(), "gemm_raw_kernel launch");
        if (rc != TANS_OK) return rc;
    }
    return hip_check(hipGetLastError(), "gemm_raw_kernel launch");
}

}  // extern "C"
