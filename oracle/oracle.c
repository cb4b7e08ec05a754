/*
 * CPU oracle for the fused tANS FP8 path.  TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as a checker or as the timed CPU baseline.
 * Nothing in the shipped package (tans-vectoradd_amd/) links or calls it.
 *
 * Contents, each restating a piece of doublewordai/tans-vectoradd:
 *   1. FP8 E4M3FN decode and round-to-nearest-even, saturate-to-finite
 *      encode, and the byte add built on them.  Restates the semantics of
 *      csrc/vecadd.cu:27-35 (add_fp8_bytes: float(a)+float(b) through the
 *      saturating __nv_fp8_e4m3 constructor) from the OCP FP8 spec, not
 *      from any vendor header.  NaN inputs give the canonical 0x7F; that
 *      choice is NOT pinned by the reference (its tests only compare fused
 *      against raw).
 *   2. The reference-format codec: pair alphabet, L = 4096, 128-stream
 *      blocks with top-aligned u32 slabs.
 *        encoder  csrc/tans_codec.cpp:22-60 (encode_one),
 *                 csrc/tans_codec.cpp:100-181 (tables, block layout)
 *        decoder  csrc/tans_decode.cu:65-155 (init_tans_ctx, tans_step,
 *                 tans_decode_kernel; output [N, K])
 *        fused    csrc/vecadd.cu:156-243 (decode A and B, compose, add;
 *                 sm tiled [N/16, K, 8], output tiled [N/16, K, 16])
 *      Used as the CPU baseline and to cross-check the table builders.
 *   3. A checker for the wave64 lane layout written by the product encoder:
 *      the same tANS step semantics (csrc/tans_decode.cu:94-123; table
 *      derived from spread + freqs as rans_vectoradd/tans_codec.py:63-87),
 *      replayed over the wave-shared word stream, with the sign/mantissa nibbles
 *      unpacked bit by bit.  It shares no code with the product.
 *   4. A checker for the packed layout of short streams (pair alphabet):
 *      the same step semantics, each lane read bit by bit from its lane
 *      pair's bits (forwards or backwards), with every count, final state
 *      and padding bit checked.  Shares no code with the product either.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* 1. FP8 E4M3FN                                                        */
/* ------------------------------------------------------------------ */

/* OCP E4M3FN: bias 7, exponent field 0 is subnormal (m/8 * 2^-6), field
 * 15 with mantissa 7 is NaN, no infinities, max finite 448. */
double ora_fp8_to_double(uint8_t b)
{
    int s = b >> 7, e = (b >> 3) & 0xF, m = b & 7;
    if (e == 15 && m == 7) return NAN;
    double v = (e == 0) ? ldexp((double)m, -9) : ldexp(8.0 + m, e - 10);
    return s ? -v : v;
}

static int is_nan_byte(uint8_t b) { return (b & 0x7F) == 0x7F; }

/* Round an exactly representable double to E4M3FN, nearest-even, with
 * saturation to +-448 for every finite magnitude above 448. */
uint8_t ora_double_to_fp8_rne_sat(double v)
{
    if (isnan(v)) return 0x7F;
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    double a = fabs(v);
    if (a > 448.0) return sign | 0x7E;
    /* quantum of the binade holding a */
    int q_exp;                       /* a is rounded to a multiple of 2^q_exp */
    if (a < ldexp(1.0, -6)) {
        q_exp = -9;                  /* subnormal spacing */
    } else {
        int e2;
        frexp(a, &e2);               /* a in [2^(e2-1), 2^e2) */
        q_exp = (e2 - 1) - 3;        /* 3 mantissa bits */
    }
    double n = ldexp(a, -q_exp);     /* exact: a has few significant bits */
    double fl = floor(n);
    double fr = n - fl;
    double r;
    if (fr > 0.5) r = fl + 1.0;
    else if (fr < 0.5) r = fl;
    else r = (fmod(fl, 2.0) == 0.0) ? fl : fl + 1.0;
    double rv = ldexp(r, q_exp);
    if (rv > 448.0) return sign | 0x7E;
    if (rv == 0.0) return sign;
    /* encode rv */
    if (rv < ldexp(1.0, -6)) {
        int m = (int)ldexp(rv, 9);   /* 1..7 */
        return sign | (uint8_t)m;
    }
    int e2;
    double fr2 = frexp(rv, &e2);     /* rv = fr2 * 2^e2, fr2 in [0.5,1) */
    int ef = (e2 - 1) + 7;
    int m = (int)(fr2 * 16.0) - 8;   /* 0..7 */
    return sign | (uint8_t)(ef << 3) | (uint8_t)m;
}

uint8_t ora_fp8_add(uint8_t a, uint8_t b)
{
    if (is_nan_byte(a) || is_nan_byte(b)) return 0x7F;
    /* the sum of two E4M3 values is exact in double */
    return ora_double_to_fp8_rne_sat(ora_fp8_to_double(a) + ora_fp8_to_double(b));
}

void ora_fp8_add_lut(uint8_t* lut /* [65536], index a*256+b */)
{
    for (int a = 0; a < 256; a++)
        for (int b = 0; b < 256; b++)
            lut[a * 256 + b] = ora_fp8_add((uint8_t)a, (uint8_t)b);
}

/* Elementwise add through a prebuilt LUT (the CPU side of a raw vecadd). */
void ora_vecadd_lut(const uint8_t* lut, const uint8_t* a, const uint8_t* b,
                    uint8_t* out, int64_t n)
{
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = lut[a[i] * 256 + b[i]];
}

static inline uint8_t compose_fp8(uint32_t exp, uint32_t sm)
{
    /* csrc/vecadd.cu:37-39 */
    return (uint8_t)(((sm & 8u) << 4) | ((exp & 0xFu) << 3) | (sm & 7u));
}

/* ------------------------------------------------------------------ */
/* 2. Reference-format codec (pair alphabet, L=4096, 128-stream blocks)  */
/* ------------------------------------------------------------------ */

#define REF_L 4096u
#define REF_BLOCK 128

typedef struct {
    uint32_t** enc;   /* enc[s][rank] = L + slot  (tans_codec.cpp:100-118) */
    uint32_t* storage;
} ref_enc_tables;

static int ref_build_enc(const int32_t* freqs, int nsym, const int32_t* spread,
                         uint32_t L, ref_enc_tables* t)
{
    t->enc = (uint32_t**)calloc((size_t)nsym, sizeof(uint32_t*));
    t->storage = (uint32_t*)calloc(L, sizeof(uint32_t));
    if (!t->enc || !t->storage) return -1;
    uint32_t off = 0;
    for (int s = 0; s < nsym; s++) {
        if (freqs[s] < 0) return -2;
        t->enc[s] = t->storage + off;
        off += (uint32_t)freqs[s];
    }
    if (off != L) return -3;
    uint32_t* counts = (uint32_t*)calloc((size_t)nsym, sizeof(uint32_t));
    for (uint32_t slot = 0; slot < L; slot++) {
        int s = spread[slot];
        if (s < 0 || s >= nsym) { free(counts); return -4; }
        t->enc[s][counts[s]++] = L + slot;
    }
    free(counts);
    return 0;
}

static void ref_free_enc(ref_enc_tables* t) { free(t->enc); free(t->storage); }

/* encode_one (tans_codec.cpp:22-60): backwards over symbols, bit-by-bit
 * LSB-first renormalisation into u32 slabs.  Writes slabs to `slabs` (may
 * be NULL to only count).  Returns the number of slabs. */
static int64_t ref_encode_one(const uint8_t* sym, int64_t n, const ref_enc_tables* t,
                              const int32_t* freqs, uint32_t L, uint32_t* slabs,
                              uint32_t* x_out, uint8_t* partial_out)
{
    uint32_t x = L, cur = 0, cnt = 0;
    int64_t ns = 0;
    for (int64_t i = n - 1; i >= 0; i--) {
        int s = sym[i];
        uint32_t f = (uint32_t)freqs[s];
        while (x >= 2u * f) {
            cur |= (x & 1u) << cnt;
            cnt++;
            if (cnt == 32u) { if (slabs) slabs[ns] = cur; ns++; cur = 0; cnt = 0; }
            x >>= 1;
        }
        x = t->enc[s][x - f];
    }
    if (partial_out) *partial_out = (uint8_t)cnt;
    if (cnt > 0u) { if (slabs) slabs[ns] = cur; ns++; }
    if (x_out) *x_out = x;
    return ns;
}

/* Per-stream slab counts; returns total compressed bytes of the block
 * layout (tans_codec.cpp:138-155), or a negative error. */
int64_t ora_ref_encode_count(const uint8_t* sym, int64_t K, int64_t N,
                             const int32_t* freqs, int nsym, const int32_t* spread,
                             int32_t* slabs_out)
{
    ref_enc_tables t;
    int rc = ref_build_enc(freqs, nsym, spread, REF_L, &t);
    if (rc) { ref_free_enc(&t); return rc; }
    for (int s = 0; s < nsym; s++) {
        /* a symbol with freq 0 would hang encode_one; refuse if present */
        if (freqs[s] == 0) {
            for (int64_t i = 0; i < K * N; i++)
                if (sym[i] == s) { ref_free_enc(&t); return -5; }
        }
    }
    #pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; k++)
        slabs_out[k] = (int32_t)ref_encode_one(sym + k * N, N, &t, freqs, REF_L,
                                               NULL, NULL, NULL);
    ref_free_enc(&t);
    int64_t nblk = (K + REF_BLOCK - 1) / REF_BLOCK, total = 0;
    for (int64_t b = 0; b < nblk; b++) {
        int32_t g = 0;
        for (int64_t k = b * REF_BLOCK; k < K && k < (b + 1) * REF_BLOCK; k++)
            if (slabs_out[k] > g) g = slabs_out[k];
        if (g == 0) g = 1;
        total += (int64_t)g * REF_BLOCK * 4;
    }
    return total;
}

int ora_ref_encode_write(const uint8_t* sym, int64_t K, int64_t N,
                         const int32_t* freqs, int nsym, const int32_t* spread,
                         const int32_t* slabs, uint8_t* comp, uint16_t* states,
                         int32_t* offsets, uint8_t* partial)
{
    ref_enc_tables t;
    int rc = ref_build_enc(freqs, nsym, spread, REF_L, &t);
    if (rc) { ref_free_enc(&t); return rc; }
    int64_t nblk = (K + REF_BLOCK - 1) / REF_BLOCK;
    int32_t* G = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nblk ? nblk : 1));
    int64_t cum = 0;
    for (int64_t b = 0; b < nblk; b++) {
        int32_t g = 0;
        for (int64_t k = b * REF_BLOCK; k < K && k < (b + 1) * REF_BLOCK; k++)
            if (slabs[k] > g) g = slabs[k];
        if (g == 0) g = 1;
        G[b] = g;
        offsets[b] = (int32_t)cum;
        cum += (int64_t)g * REF_BLOCK * 4;
    }
    offsets[nblk] = (int32_t)cum;
    memset(comp, 0, (size_t)cum);
    #pragma omp parallel
    {
        uint32_t* buf = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(N + 8));
        #pragma omp for schedule(static)
        for (int64_t k = 0; k < K; k++) {
            uint32_t x; uint8_t p;
            int64_t ns = ref_encode_one(sym + k * N, N, &t, freqs, REF_L, buf, &x, &p);
            states[k] = (uint16_t)x;
            partial[k] = p;
            int64_t b = k / REF_BLOCK, tid = k % REF_BLOCK;
            for (int64_t g = 0; g < ns; g++) {
                int64_t row = G[b] - ns + g;          /* top-aligned */
                memcpy(comp + offsets[b] + row * REF_BLOCK * 4 + tid * 4, &buf[g], 4);
            }
        }
        free(buf);
    }
    free(G);
    ref_free_enc(&t);
    return 0;
}

/* Reference decoder state (tans_decode.cu:14-21). */
typedef struct { uint32_t x, hi, lo, cnt; int slab_idx; int64_t base_u32; } ref_ctx;

static void ref_init(ref_ctx* c, const uint32_t* comp, const int32_t* offsets,
                     const uint16_t* states, const uint8_t* partial,
                     int64_t blk, int64_t sid, int64_t tid)
{
    /* tans_decode.cu:65-92 */
    int32_t base = offsets[blk], next = offsets[blk + 1];
    int spb = (next - base) / (REF_BLOCK * 4);
    c->x = states[sid];
    c->base_u32 = base / 4;
    int top = spb - 1, next_top = spb - 2;
    c->hi = comp[c->base_u32 + (int64_t)top * REF_BLOCK + tid];
    c->lo = next_top >= 0 ? comp[c->base_u32 + (int64_t)next_top * REF_BLOCK + tid] : 0u;
    c->slab_idx = next_top - 1;
    uint32_t p = partial[sid];
    c->cnt = p == 0u ? 0u : 32u - p;
}

static inline uint8_t ref_step(ref_ctx* c, const uint32_t* comp, int64_t tid,
                               const uint32_t* tbl)
{
    /* tans_decode.cu:94-123 */
    uint32_t e = tbl[c->x - REF_L];
    uint32_t nb = (e >> 8) & 0xFu, base_state = (e >> 16) & 0xFFFFu;
    uint8_t sym = (uint8_t)(e & 0xFFu);
    uint64_t cat = ((uint64_t)c->hi << 32) | c->lo;
    uint32_t shifted = (uint32_t)((cat << (c->cnt & 31u)) >> 32);  /* __funnelshift_l */
    uint32_t bits = nb == 0u ? 0u : shifted >> (32u - nb);
    c->x = base_state | bits;
    c->cnt += nb;
    if (c->cnt >= 32u) {
        c->cnt -= 32u;
        c->hi = c->lo;
        if (c->slab_idx >= 0) {
            c->lo = comp[c->base_u32 + (int64_t)c->slab_idx * REF_BLOCK + tid];
            c->slab_idx -= 1;
        } else {
            c->lo = 0u;
        }
    }
    return sym;
}

/* Standalone decode, output [N, K] (tans_decode.cu:125-155). */
int ora_ref_decode(const uint8_t* comp8, const int32_t* offsets, const uint16_t* states,
                   const uint8_t* partial, const uint8_t* sm /* [N/2, K] */,
                   const uint32_t* tbl /* [4096] */, int64_t K, int64_t N,
                   uint8_t* out /* [N, K] */)
{
    const uint32_t* comp = (const uint32_t*)comp8;
    #pragma omp parallel for schedule(static)
    for (int64_t sid = 0; sid < K; sid++) {
        ref_ctx c;
        int64_t blk = sid / REF_BLOCK, tid = sid % REF_BLOCK;
        ref_init(&c, comp, offsets, states, partial, blk, sid, tid);
        for (int64_t i = 0; i < N / 2; i++) {
            uint8_t s = ref_step(&c, comp, tid, tbl);
            uint8_t m = sm[i * K + sid];
            out[(2 * i) * K + sid] = compose_fp8(s >> 4, m & 0xFu);
            out[(2 * i + 1) * K + sid] = compose_fp8(s & 0xFu, m >> 4);
        }
    }
    return 0;
}

/* Fused decode + add over two reference-format encodings, tiled output
 * (vecadd.cu:156-243).  `lut` is ora_fp8_add_lut's table. */
/* Threads used by the OpenMP loops above (the CPU baseline is timed with
 * all host cores and with one). */
void ora_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

int ora_ref_decode_add(const uint8_t* a_comp8, const int32_t* a_off, const uint16_t* a_st,
                       const uint8_t* a_part, const uint8_t* a_sm,
                       const uint8_t* b_comp8, const int32_t* b_off, const uint16_t* b_st,
                       const uint8_t* b_part, const uint8_t* b_sm,
                       const uint32_t* tbl, const uint8_t* lut,
                       int64_t K, int64_t N, uint8_t* out)
{
    const uint32_t* ac = (const uint32_t*)a_comp8;
    const uint32_t* bc = (const uint32_t*)b_comp8;
    int64_t n_tiles = (N / 2) / 8;
    #pragma omp parallel for schedule(static)
    for (int64_t sid = 0; sid < K; sid++) {
        ref_ctx ca, cb;
        int64_t blk = sid / REF_BLOCK, tid = sid % REF_BLOCK;
        ref_init(&ca, ac, a_off, a_st, a_part, blk, sid, tid);
        ref_init(&cb, bc, b_off, b_st, b_part, blk, sid, tid);
        for (int64_t t = 0; t < n_tiles; t++) {
            const uint8_t* sa = a_sm + (t * K + sid) * 8;
            const uint8_t* sb = b_sm + (t * K + sid) * 8;
            uint8_t* o = out + (t * K + sid) * 16;
            for (int p = 0; p < 8; p++) {
                uint8_t ya = ref_step(&ca, ac, tid, tbl);
                uint8_t yb = ref_step(&cb, bc, tid, tbl);
                uint8_t a0 = compose_fp8(ya >> 4, sa[p] & 0xFu), a1 = compose_fp8(ya & 0xFu, sa[p] >> 4);
                uint8_t b0 = compose_fp8(yb >> 4, sb[p] & 0xFu), b1 = compose_fp8(yb & 0xFu, sb[p] >> 4);
                o[2 * p] = lut[a0 * 256 + b0];
                o[2 * p + 1] = lut[a1 * 256 + b1];
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* 3. Checker for the wave64 lane layout                               */
/* ------------------------------------------------------------------ */

/* Layout being checked (written by the product encoder):
 *   lanes are the K rows of the input; lane k belongs to group g = k/64 at
 *   column j = k%64.  Each lane's decode-order bits are cut into u32 words
 *   (LSB = earliest bit); each decode step reads nb bits as one value.
 *   Group g's words form one stream at comp_words[offsets[g] ..], in the
 *   order of this refill schedule: first every active lane (ascending j)
 *   takes one word, then every active lane takes a second; the steps are
 *   cut into segments, and after each segment except the last, each active
 *   lane (ascending j) holding at most 32 unread bits takes the next stream
 *   word (+32 bits); after the second-to-last segment only a lane holding
 *   fewer bits than the last segment can read does, unless the last tile of
 *   16 elements (16/sps steps) holds that last segment alone: then that
 *   check is the plain one.  Segments: with
 *   2^11-state tables (whose symbols all have f >= 2, so nb <= 10), every 8
 *   steps are cut into 3, 3 and 2 steps, and the last segment can read
 *   10 bits per step; with other tables, step pairs (2p, 2p+1), and the
 *   last one can read 24 bits.
 *   states[k] is the initial decoder state in [L, 2L).
 *   Symbols: sps=2 -> pair symbol e0*16+e1 per step; sps=1 -> one exponent.
 *   Sign/mantissa: tiles of 16 elements, 8 bytes per (tile, lane) at
 *   sm[(t*K + k)*8]; u32 word h covers elements 8h..8h+7 of the tile:
 *   element i<4: sign bit 8i+7, mantissa bits 8i..8i+2;
 *   element 4+i: mantissa bits 8i+4..8i+6, sign bit 8((i+1)%4)+3.
 * Returns 0 on success, or a negative code naming the first inconsistency
 * (-10 bad state, -11 final state != L, -12 stream overrun,
 *  -13 nonzero unread bits, -14 nonzero stream padding, -15 no memory). */
static uint32_t sm_nibble_of(const uint8_t* sm8, int e /* 0..15 */)
{
    uint32_t w;
    memcpy(&w, sm8 + (e / 8) * 4, 4);
    int i = e % 8;
    uint32_t sign, mant;
    if (i < 4) {
        sign = (w >> (8 * i + 7)) & 1u;
        mant = (w >> (8 * i)) & 7u;
    } else {
        i -= 4;
        mant = (w >> (8 * i + 4)) & 7u;
        sign = (w >> (8 * ((i + 1) % 4) + 3)) & 1u;
    }
    return (sign << 3) | mant;
}

typedef struct {
    uint32_t* words;     /* words received so far */
    int64_t n_words, cap;
    uint64_t rd;         /* bits consumed */
    uint32_t x;
} w64_lane;

static int lane_take(w64_lane* ln, uint32_t w)
{
    if (ln->n_words == ln->cap) {
        int64_t nc = ln->cap ? 2 * ln->cap : 64;
        uint32_t* p = (uint32_t*)realloc(ln->words, sizeof(uint32_t) * (size_t)nc);
        if (!p) return -15;
        ln->words = p; ln->cap = nc;
    }
    ln->words[ln->n_words++] = w;
    return 0;
}

static uint32_t lane_read(w64_lane* ln, int nb)
{
    uint32_t v = 0;
    for (int b = 0; b < nb; b++, ln->rd++) {
        uint32_t w = ln->words[ln->rd / 32];
        v |= ((w >> (ln->rd % 32)) & 1u) << b;
    }
    return v;
}

int ora_w64_decode(const uint8_t* comp8, const int64_t* offsets, const uint16_t* states,
                   const uint8_t* sm, const int32_t* spread, const int32_t* freqs,
                   int nsym, int log2L, int sps, int64_t K, int64_t N,
                   uint8_t* out /* [K, N] row-major */)
{
    const uint32_t* comp = (const uint32_t*)comp8;
    uint32_t L = 1u << log2L;
    /* slot -> (sym, nb, base) from spread + freqs, rans_vectoradd/tans_codec.py:63-87 */
    int32_t* t_sym = (int32_t*)malloc(sizeof(int32_t) * L);
    int32_t* t_nb = (int32_t*)malloc(sizeof(int32_t) * L);
    uint32_t* t_base = (uint32_t*)malloc(sizeof(uint32_t) * L);
    int64_t* counts = (int64_t*)calloc((size_t)nsym, sizeof(int64_t));
    for (uint32_t slot = 0; slot < L; slot++) {
        int s = spread[slot];
        uint32_t xp = (uint32_t)freqs[s] + (uint32_t)counts[s]++;
        int nb = 0;
        uint32_t v = xp;
        while (v < L) { v <<= 1; nb++; }
        t_sym[slot] = s; t_nb[slot] = nb; t_base[slot] = xp << nb;
    }
    free(counts);
    const int64_t steps = (sps == 2) ? N / 2 : N;
    const int64_t n_groups = (K + 63) / 64;
    int err = 0;
    #pragma omp parallel for schedule(dynamic, 1) reduction(min:err)
    for (int64_t g = 0; g < n_groups; g++) {
        int lanes = (int)((K - g * 64) < 64 ? (K - g * 64) : 64);
        w64_lane ln[64];
        memset(ln, 0, sizeof(ln));
        int bad = 0;
        for (int j = 0; j < lanes; j++) {
            ln[j].x = states[g * 64 + j];
            if (ln[j].x < L || ln[j].x >= 2 * L) bad = -10;
        }
        int64_t pos = offsets[g], end = offsets[g + 1];
        if (steps > 0) {
            for (int r = 0; r < 2 && !bad; r++)
                for (int j = 0; j < lanes && !bad; j++) {
                    if (pos >= end) { bad = -12; break; }
                    if (lane_take(&ln[j], comp[pos++])) bad = -15;
                }
        }
        /* segment of each step and the number of segments (see above) */
        const int triple = (log2L == 11);
        #define SEG_OF(i) (triple ? 3 * ((i) / 8) + ((i) % 8 < 3 ? 0 : (i) % 8 < 6 ? 1 : 2) : (i) / 2)
        const int64_t n_seg = steps > 0 ? SEG_OF(steps - 1) + 1 : 0;
        int64_t last_start = steps - 1;       /* first step of the last segment */
        while (last_start > 0 && SEG_OF(last_start - 1) == n_seg - 1) last_start--;
        /* a last 16-element tile of one segment makes the final check the plain one */
        const int64_t tile_steps = 16 / sps;
        const int one_seg_tile = steps > tile_steps && last_start == tile_steps * ((steps - 1) / tile_steps);
        const uint64_t final_below = one_seg_tile ? 33 : triple ? (uint64_t)(10 * (steps - last_start)) : 24;
        for (int64_t i = 0; i < steps && !bad; i++) {
            for (int j = 0; j < lanes && !bad; j++) {
                int64_t k = g * 64 + j;
                uint32_t slot = ln[j].x - L;
                int s = t_sym[slot], nb = t_nb[slot];
                ln[j].x = t_base[slot] + lane_read(&ln[j], nb);
                int e0 = (sps == 2) ? (s >> 4) : s, e1 = s & 0xF;
                int64_t el = (sps == 2) ? 2 * i : i;
                const uint8_t* sm8 = sm + ((el / 16) * K + k) * 8;
                out[k * N + el] = compose_fp8((uint32_t)e0, sm_nibble_of(sm8, (int)(el % 16)));
                if (sps == 2)
                    out[k * N + el + 1] = compose_fp8((uint32_t)e1, sm_nibble_of(sm8, (int)((el + 1) % 16)));
            }
            const int64_t p = SEG_OF(i);
            const int seg_end = i == steps - 1 || SEG_OF(i + 1) != p;
            if (seg_end && p + 1 < n_seg) {
                const uint64_t below = (p + 2 == n_seg) ? final_below : 33;
                for (int j = 0; j < lanes && !bad; j++) {
                    uint64_t avail = (uint64_t)ln[j].n_words * 32 - ln[j].rd;
                    if (avail < below) {
                        if (pos >= end) { bad = -12; break; }
                        if (lane_take(&ln[j], comp[pos++])) bad = -15;
                    }
                }
            }
        }
        #undef SEG_OF
        for (int j = 0; j < lanes && !bad; j++) {
            if (ln[j].x != L) { bad = -11; break; }
            for (uint64_t p = ln[j].rd; p < (uint64_t)ln[j].n_words * 32; p++)
                if ((ln[j].words[p / 32] >> (p % 32)) & 1u) { bad = -13; break; }
        }
        for (int64_t p = pos; p < end && !bad; p++)
            if (comp[p]) bad = -14;
        for (int j = 0; j < 64; j++) free(ln[j].words);
        if (bad) err = bad;
    }
    free(t_sym); free(t_nb); free(t_base);
    return err;
}

/* ------------------------------------------------------------------ */
/* 4. Checker for the packed layout of short streams                  */
/* ------------------------------------------------------------------ */

/* Layout being checked (written by the product encoder for the pair
 * alphabet, L = 4096, at most 32 steps per lane):
 *   group g's stream starts at byte 4*offsets[g]: 32 lane-pair bit counts
 *   (1 byte each when N <= 16, else 2, little-endian), then a bit area
 *   (bit b = bit b%8 of byte b/8 of the area).  Pair p = lanes 2p, 2p+1
 *   owns bits [S_p, E_p), S_p = sum of the counts before p, E_p = S_p +
 *   count_p.  A lane's bits in decode order: its initial state minus L
 *   (12 bits), then each step's nb bits, every value LSB first.  The even
 *   lane's i-th bit is at S_p + i, the odd lane's at E_p - 1 - i.  Lanes
 *   past K count 0 bits; the rest of the stream is zero.
 *   Sign/mantissa tiles as in section 3.
 * Returns 0, or a negative code naming the first inconsistency: -11 final
 * state != L, -12 a lane reads outside its pair's bits, -13 the pair's
 * two lanes do not use its count exactly, -14 nonzero bits past the
 * counts, -16 a lane past K with a nonzero count, -17 counts overrun the
 * stream. */
typedef struct {
    const uint8_t* area;
    int64_t lo, hi;     /* the pair's bits [lo, hi) */
    int64_t at;         /* next bit (even: at, going up; odd: at - 1, going down) */
    int dir;            /* +1 even lane, -1 odd lane */
    int err;
} pk_reader;

static uint32_t pk_read(pk_reader* r, int nb)
{
    uint32_t v = 0;
    for (int b = 0; b < nb; b++) {
        int64_t pos = r->dir > 0 ? r->at : r->at - 1;
        if (pos < r->lo || pos >= r->hi) { r->err = -12; return 0; }
        v |= (uint32_t)((r->area[pos >> 3] >> (pos & 7)) & 1u) << b;
        r->at += r->dir;
    }
    return v;
}

int ora_packed_decode(const uint8_t* comp8, const int64_t* offsets, const uint8_t* sm,
                      const int32_t* spread, const int32_t* freqs, int64_t K, int64_t N,
                      uint8_t* out /* [K, N] row-major */)
{
    const uint32_t L = 4096;
    int32_t* t_sym = (int32_t*)malloc(sizeof(int32_t) * L);
    int32_t* t_nb = (int32_t*)malloc(sizeof(int32_t) * L);
    uint32_t* t_base = (uint32_t*)malloc(sizeof(uint32_t) * L);
    int64_t* counts = (int64_t*)calloc(256, sizeof(int64_t));
    for (uint32_t slot = 0; slot < L; slot++) {
        int s = spread[slot];
        uint32_t xp = (uint32_t)freqs[s] + (uint32_t)counts[s]++;
        int nb = 0;
        uint32_t v = xp;
        while (v < L) { v <<= 1; nb++; }
        t_sym[slot] = s; t_nb[slot] = nb; t_base[slot] = xp << nb;
    }
    free(counts);
    const int64_t steps = N / 2;
    const int hb = steps <= 8 ? 1 : 2;
    const int64_t n_groups = (K + 63) / 64;
    int err = 0;
    #pragma omp parallel for schedule(dynamic, 4) reduction(min:err)
    for (int64_t g = 0; g < n_groups; g++) {
        const uint8_t* st = comp8 + offsets[g] * 4;
        const int64_t bytes = (offsets[g + 1] - offsets[g]) * 4;
        const int lanes = (int)((K - g * 64) < 64 ? (K - g * 64) : 64);
        int bad = 0;
        int64_t cnt[32], start[33];
        start[0] = 0;
        if (bytes < 32 * hb) bad = -17;
        for (int p = 0; p < 32 && !bad; p++) {
            cnt[p] = st[p * hb] | (hb == 2 ? (int64_t)st[p * hb + 1] << 8 : 0);
            start[p + 1] = start[p] + cnt[p];
            if (2 * p >= lanes && cnt[p]) bad = -16;
        }
        if (!bad && (start[32] + 7) / 8 > bytes - 32 * hb) bad = -17;
        const uint8_t* area = st + 32 * hb;
        for (int p = 0; p < 32 && !bad; p++) {
            int64_t used = 0;
            for (int side = 0; side < 2 && !bad; side++) {
                const int j = 2 * p + side;
                if (j >= lanes) continue;
                const int64_t k = g * 64 + j;
                pk_reader r = {area, start[p], start[p + 1], side ? start[p + 1] : start[p],
                               side ? -1 : 1, 0};
                uint32_t x = L + pk_read(&r, 12);
                for (int64_t i = 0; i < steps && !r.err; i++) {
                    uint32_t slot = x - L;
                    int s = t_sym[slot];
                    x = t_base[slot] + pk_read(&r, t_nb[slot]);
                    const int64_t el = 2 * i;
                    const uint8_t* sm8 = sm + ((el / 16) * K + k) * 8;
                    out[k * N + el] = compose_fp8((uint32_t)(s >> 4), sm_nibble_of(sm8, (int)(el % 16)));
                    out[k * N + el + 1] = compose_fp8((uint32_t)(s & 0xF), sm_nibble_of(sm8, (int)((el + 1) % 16)));
                }
                if (r.err) { bad = r.err; break; }
                if (x != L) { bad = -11; break; }
                used += side ? start[p + 1] - r.at : r.at - start[p];
            }
            if (!bad && used != cnt[p]) bad = -13;
        }
        for (int64_t b = start[32]; b < (bytes - 32 * hb) * 8 && !bad; b++)
            if ((area[b >> 3] >> (b & 7)) & 1u) bad = -14;
        if (bad) err = bad;
    }
    free(t_sym); free(t_nb); free(t_base);
    return err;
}
