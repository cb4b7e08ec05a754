// CPU side of the MI355X tANS FP8 library: nibble split, decode-table
// construction and the encoder into the wave64 lane layout (format described
// in include/tans_amd.h).
//
// The encoder follows the tANS construction of csrc/tans_codec.cpp:22-60
// (walk the symbols backwards from x = L, renormalise the state into
// [f_s, 2 f_s) by emitting its low bits, then x = L + slot of the
// rank-th occurrence of s in the spread, tans_codec.cpp:100-118).  What
// differs is the bit order and layout: the bits of each step are kept as one
// chunk, the chunks are written forwards in decode order LSB-first, and the
// lanes of a 64-lane group are interleaved word by word in rows, so a wave's
// refills hit a few adjacent 256-byte rows.  There is no partial-slab count:
// a lane's bitstream starts at bit 0 of its first word.
#include "../../include/tans_amd.h"
#include "schedule.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

thread_local std::string g_err;

int fail(int code, const char* msg) {
    g_err = msg;
    return code;
}

inline uint32_t rotl32(uint32_t v, int r) { return (v << r) | (v >> (32 - r)); }

inline int ilog2(uint32_t v) { return 31 - __builtin_clz(v); }

// Refill schedule shared with the decoders (schedule.h): every lane starts
// with two 32-bit words of its group's stream (the first words of lanes 0,
// 1, ..., then their second words).  After each segment of steps but the
// last (two steps; three, three and two with 2^11-state tables), a lane
// holding at most 32 unread bits takes the next word (lanes in ascending
// order); after the second-to-last segment only a lane holding fewer bits
// than the last segment can read does.  A segment reads at most 30 bits, so
// the 64-bit buffer never runs dry and never overflows.
// Zero words appended after the last group, so 16-byte segment loads near
// the end stay inside the buffer.
constexpr int64_t kTailWords = 256;

struct EncTables {
    std::vector<uint32_t> start;   // start[s]: first index of s in next
    std::vector<uint32_t> next;    // next[start[s] + rank] = L + slot
    std::vector<uint32_t> freq;
};

int build_enc_tables(const int32_t* freqs, int32_t nsym, const int32_t* spread,
                     int32_t log2L, EncTables& t) {
    const uint32_t L = 1u << log2L;
    t.start.assign(nsym, 0);
    t.freq.assign(nsym, 0);
    t.next.assign(L, 0);
    const bool triple = log2L == tans_sched::kTripleLog2L;
    uint64_t sum = 0;
    for (int s = 0; s < nsym; s++) {
        if (freqs[s] < 0) return fail(TANS_ETABLE, "negative frequency");
        if (triple && freqs[s] > 0 && (uint32_t)freqs[s] < tans_sched::kTripleMinFreq)
            return fail(TANS_ETABLE, "tables of 2^11 states need every present symbol's "
                                     "frequency >= 2 (nb <= 10)");
        t.start[s] = (uint32_t)sum;
        t.freq[s] = (uint32_t)freqs[s];
        sum += (uint32_t)freqs[s];
    }
    if (sum != L) return fail(TANS_ETABLE, "freqs must sum to L = 2^log2L");
    std::vector<uint32_t> cnt(nsym, 0);
    for (uint32_t slot = 0; slot < L; slot++) {
        int s = spread[slot];
        if (s < 0 || s >= nsym) return fail(TANS_ETABLE, "spread symbol out of range");
        if (cnt[s] >= t.freq[s]) return fail(TANS_ETABLE, "spread disagrees with freqs");
        t.next[t.start[s] + cnt[s]++] = L + slot;
    }
    return TANS_OK;
}

// Encode one lane of S symbols.  chunk[i] receives step i's bits (low 16)
// and nb (bits 16+).  words receives the decode-order bitstream, LSB first
// (room for ceil(S*log2L/32)+1 words).  Returns the word count, or -1 if a
// symbol lies outside the alphabet or has frequency 0.
int64_t encode_lane(const uint8_t* sym, int64_t S, const EncTables& t, uint32_t L,
                    uint32_t* chunk, uint32_t* words, uint32_t* x0) {
    uint32_t x = L;
    const uint32_t* freq = t.freq.data();
    const uint32_t* start = t.start.data();
    const uint32_t* next = t.next.data();
    const uint32_t nsym = (uint32_t)t.freq.size();
    for (int64_t i = S - 1; i >= 0; i--) {
        const uint32_t s = sym[i];
        if (s >= nsym) return -1;
        const uint32_t f = freq[s];
        if (f == 0) return -1;
        // nb such that (x >> nb) lies in [f, 2f)
        int nb = ilog2(x) - ilog2(f);
        if ((x >> nb) < f) nb--;
        chunk[i] = (x & ((1u << nb) - 1u)) | ((uint32_t)nb << 16);
        x = next[start[s] + (x >> nb) - f];
    }
    *x0 = x;
    uint64_t acc = 0;
    int n = 0;
    int64_t nw = 0;
    for (int64_t i = 0; i < S; i++) {
        acc |= (uint64_t)(chunk[i] & 0xFFFFu) << n;
        n += (int)(chunk[i] >> 16);
        if (n >= 32) {
            words[nw++] = (uint32_t)acc;
            acc >>= 32;
            n -= 32;
        }
    }
    if (n > 0) words[nw++] = (uint32_t)acc;
    return nw;
}

struct EncodeHandle {
    int64_t K = 0, S = 0, n_groups = 0, total_words = 0;
    bool packed = false;                          // packed layout: no states
    std::vector<std::vector<uint32_t>> streams;   // per group, 4-word padded
    std::vector<uint16_t> states;
};

// Bit writer of the packed layout's area (bit b = bit b % 8 of byte b / 8).
inline void put_bit(uint8_t* area, int64_t b, uint32_t v) {
    area[b >> 3] |= (uint8_t)((v & 1u) << (b & 7));
}

// One group of the packed layout (schedule.h, tans_pack): lanes' bits in
// decode order are the state minus L and each step's chunk; even lanes
// forwards from their pair's start, odd lanes backwards from its end.
void pack_group(const uint32_t* chunk, const uint32_t* x0, int lanes, int64_t S, uint32_t L,
                std::vector<uint32_t>& out) {
    const int hb = tans_pack::hdr_bytes(S);
    int64_t len[TANS_LANES] = {0};
    for (int j = 0; j < lanes; j++) {
        len[j] = tans_pack::kStateBits;
        for (int64_t i = 0; i < S; i++) len[j] += (int64_t)(chunk[j * S + i] >> 16);
    }
    int64_t total = 0;
    for (int j = 0; j < TANS_LANES; j++) total += len[j];
    const int64_t bytes = (tans_pack::hdr_total(S) + (total + 7) / 8 + 15) / 16 * 16;
    std::vector<uint8_t> buf((size_t)bytes, 0);
    for (int p = 0; p < tans_pack::kPairs; p++) {
        const uint32_t n = (uint32_t)(len[2 * p] + len[2 * p + 1]);
        for (int b = 0; b < hb; b++) buf[(size_t)(p * hb + b)] = (uint8_t)(n >> (8 * b));
    }
    uint8_t* area = buf.data() + tans_pack::hdr_total(S);
    int64_t start = 0;
    for (int p = 0; p < tans_pack::kPairs; p++) {
        const int64_t end = start + len[2 * p] + len[2 * p + 1];
        for (int side = 0; side < 2; side++) {
            const int j = 2 * p + side;
            if (j >= lanes) break;
            // bit i of the lane goes to start + i (even) or end - 1 - i (odd)
            int64_t i = 0;
            auto put = [&](uint32_t v, int nb) {
                for (int b = 0; b < nb; b++, i++)
                    put_bit(area, side ? end - 1 - i : start + i, v >> b);
            };
            put(x0[j] - L, tans_pack::kStateBits);
            for (int64_t s = 0; s < S; s++) {
                const uint32_t c = chunk[j * S + s];
                put(c & 0xFFFFu, (int)(c >> 16));
            }
        }
        start = end;
    }
    out.assign((size_t)(bytes / 4), 0u);
    std::memcpy(out.data(), buf.data(), (size_t)bytes);
}

}  // namespace

extern "C" {

const char* tans_last_error(void) { return g_err.c_str(); }

void tans_internal_set_error(const char* msg) { g_err = msg ? msg : ""; }

// The refill thresholds after segment j of a stream of S steps (schedule.h):
// the one the encoders apply (which = 0) and the one the GPU decoders'
// placement of checks amounts to (which = 1); 0 = no check.  Not part of the
// public ABI: the CPU tests compare the two.
int tans_internal_check_below(int32_t which, int64_t S, int32_t triple, int64_t j) {
    return which ? tans_sched::decoder_below(S, triple != 0, j)
                 : tans_sched::encoder_below(S, triple != 0, j);
}

int tans_split_fp8(const uint8_t* fp8, int64_t K, int64_t N, int32_t sps,
                   uint8_t* symbols, uint8_t* sm) {
    if ((!fp8 && K * N != 0) || K < 0 || N < 0 || (N % 2) != 0)
        return fail(TANS_EINVAL, "split: need K >= 0 and even N >= 0");
    if (sps != 1 && sps != 2) return fail(TANS_EINVAL, "split: sps must be 1 or 2");
    const int64_t S = N / sps;
    const int64_t n_tiles = (N + TANS_TILE - 1) / TANS_TILE;
    #pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; k++) {
        const uint8_t* row = fp8 + k * N;
        uint8_t* srow = symbols + k * S;
        if (sps == 2) {
            for (int64_t i = 0; i < S; i++)
                srow[i] = (uint8_t)((((row[2 * i] >> 3) & 0xF) << 4) | ((row[2 * i + 1] >> 3) & 0xF));
        } else {
            for (int64_t i = 0; i < S; i++) srow[i] = (uint8_t)((row[i] >> 3) & 0xF);
        }
        for (int64_t t = 0; t < n_tiles; t++) {
            uint8_t tile[TANS_TILE] = {0};
            int64_t m = std::min<int64_t>(TANS_TILE, N - t * TANS_TILE);
            std::memcpy(tile, row + t * TANS_TILE, (size_t)m);
            uint32_t w[2];
            for (int h = 0; h < 2; h++) {
                uint32_t a, b;
                std::memcpy(&a, tile + 8 * h, 4);
                std::memcpy(&b, tile + 8 * h + 4, 4);
                w[h] = (a & 0x87878787u) | rotl32(b & 0x87878787u, 4);
            }
            std::memcpy(sm + (t * K + k) * 8, w, 8);
        }
    }
    return TANS_OK;
}

int tans_build_decode_table(const int32_t* spread, const int32_t* freqs, int32_t nsym,
                            int32_t log2L, uint32_t* table) {
    if (!spread || !freqs || !table) return fail(TANS_EINVAL, "table: null pointer");
    if (!((nsym == 256 && log2L == TANS_PAIR_LOG2L) || (nsym == 16 && log2L == TANS_NIBBLE_LOG2L)))
        return fail(TANS_EINVAL, "table: need (nsym 256, log2L 12) or (nsym 16, log2L 11)");
    EncTables t;
    int rc = build_enc_tables(freqs, nsym, spread, log2L, t);   // validates
    if (rc) return rc;
    const uint32_t L = 1u << log2L;
    std::vector<uint32_t> cnt(nsym, 0);
    for (uint32_t slot = 0; slot < L; slot++) {
        const uint32_t s = (uint32_t)spread[slot];
        const uint32_t xp = t.freq[s] + cnt[s]++;
        const int nb = log2L - ilog2(xp);
        const uint32_t base = xp << nb;
        const uint32_t ex = (nsym == 256) ? (((s >> 4) << 11) | ((s & 0xF) << 19)) : (s << 11);
        table[2 * slot] = (uint32_t)nb | ex | ((uint32_t)nb << 27);
        table[2 * slot + 1] = (base - L) * 8u;
    }
    return TANS_OK;
}

int tans_build_encode_table(const int32_t* spread, const int32_t* freqs, int32_t nsym,
                            int32_t log2L, uint32_t* enc_tab, uint16_t* enc_next) {
    if (!spread || !freqs || !enc_tab || !enc_next) return fail(TANS_EINVAL, "encode table: null pointer");
    if (!((nsym == 256 && log2L == TANS_PAIR_LOG2L) || (nsym == 16 && log2L == TANS_NIBBLE_LOG2L)))
        return fail(TANS_EINVAL, "encode table: need (nsym 256, log2L 12) or (nsym 16, log2L 11)");
    EncTables t;
    int rc = build_enc_tables(freqs, nsym, spread, log2L, t);   // validates
    if (rc) return rc;
    for (int s = 0; s < nsym; s++) enc_tab[s] = t.freq[(size_t)s] | (t.start[(size_t)s] << 16);
    for (uint32_t i = 0; i < (1u << log2L); i++) enc_next[i] = (uint16_t)t.next[i];
    return TANS_OK;
}

}  // extern "C"

namespace {

int encode_begin(const uint8_t* symbols, int64_t K, int64_t S, const int32_t* freqs,
                 int32_t nsym, const int32_t* spread, int32_t log2L, bool packed, void** handle,
                 int64_t* comp_bytes, int64_t* n_offsets) {
    if (!handle || !comp_bytes || !n_offsets) return fail(TANS_EINVAL, "encode: null output");
    *handle = nullptr;
    if (K < 0 || S < 0 || (!symbols && K * S != 0) || !freqs || !spread)
        return fail(TANS_EINVAL, "encode: bad shape or null input");
    if (log2L < 1 || log2L > 12) return fail(TANS_EINVAL, "encode: log2L must be in [1, 12]");
    if (nsym < 1 || nsym > 256) return fail(TANS_EINVAL, "encode: nsym must be in [1, 256]");
    if (packed && (log2L != TANS_PAIR_LOG2L || S < 1 || S > tans_pack::kMaxSteps))
        return fail(TANS_EINVAL, "encode_packed: needs a 2^12-state table and 1..32 steps per lane");
    EncTables t;
    int rc = build_enc_tables(freqs, nsym, spread, log2L, t);
    if (rc) return rc;
    const uint32_t L = 1u << log2L;
    EncodeHandle* h = new (std::nothrow) EncodeHandle;
    if (!h) return fail(TANS_ENOMEM, "encode: out of memory");
    h->K = K;
    h->S = S;
    h->packed = packed;
    h->n_groups = (K + TANS_LANES - 1) / TANS_LANES;
    try {
        h->streams.resize((size_t)h->n_groups);
        h->states.assign((size_t)K, 0);
    } catch (...) {
        delete h;
        return fail(TANS_ENOMEM, "encode: out of memory");
    }
    const int64_t max_words = (S * (int64_t)log2L + 31) / 32 + 1;
    int bad_symbol = 0;
    #pragma omp parallel
    {
        std::vector<uint32_t> chunk((size_t)std::max<int64_t>(S, 1) * TANS_LANES);
        std::vector<uint32_t> words((size_t)(TANS_LANES * max_words));
        std::vector<int64_t> nw(TANS_LANES), taken(TANS_LANES);
        std::vector<int32_t> cnt(TANS_LANES);
        std::vector<uint32_t> x0s(TANS_LANES);
        #pragma omp for schedule(dynamic, 4)
        for (int64_t g = 0; g < h->n_groups; g++) {
            const int lanes = (int)std::min<int64_t>(TANS_LANES, K - g * TANS_LANES);
            bool ok = true;
            for (int j = 0; j < lanes; j++) {
                const int64_t k = g * TANS_LANES + j;
                uint32_t x0;
                nw[j] = encode_lane(symbols + k * S, S, t, L, chunk.data() + j * S,
                                    words.data() + j * max_words, &x0);
                if (nw[j] < 0) { ok = false; break; }
                h->states[(size_t)k] = (uint16_t)x0;
                x0s[j] = x0;
            }
            if (!ok) {
                #pragma omp atomic write
                bad_symbol = 1;
                continue;
            }
            std::vector<uint32_t>& out = h->streams[(size_t)g];
            if (packed) {
                pack_group(chunk.data(), x0s.data(), lanes, S, L, out);
                continue;
            }
            // Replay the decoders' refill schedule to order the words.
            out.clear();
            out.reserve((size_t)(lanes * (max_words + 3)));
            auto take = [&](int j) {
                const int64_t r = taken[j]++;
                out.push_back(r < nw[j] ? words[(size_t)(j * max_words + r)] : 0u);
                cnt[j] += 32;
            };
            for (int j = 0; j < lanes; j++) { cnt[j] = 0; taken[j] = 0; }
            if (S > 0) {
                for (int r = 0; r < 2; r++)
                    for (int j = 0; j < lanes; j++) take(j);
            }
            const bool triple = log2L == tans_sched::kTripleLog2L;
            const int64_t n_seg = tans_sched::segments(S, triple);
            for (int64_t q = 0; q + 1 < n_seg; q++) {
                const int32_t below = tans_sched::encoder_below(S, triple, q);
                const int64_t i0 = tans_sched::seg_start(q, triple);
                const int64_t i1 = tans_sched::seg_start(q + 1, triple);
                for (int j = 0; j < lanes; j++) {
                    const uint32_t* ch = chunk.data() + j * S;
                    for (int64_t i = i0; i < i1; i++) cnt[j] -= (int32_t)(ch[i] >> 16);
                    if (cnt[j] < below) take(j);
                }
            }
            while (out.size() % 4) out.push_back(0u);
        }
    }
    if (bad_symbol) {
        delete h;
        return fail(TANS_ESYMBOL, "encode: data holds a symbol outside the alphabet or with frequency 0");
    }
    int64_t total = 0;
    for (const auto& st : h->streams) total += (int64_t)st.size();
    h->total_words = total;
    *comp_bytes = (total + kTailWords) * 4;
    *n_offsets = h->n_groups + 1;
    *handle = h;
    return TANS_OK;
}

}  // namespace

extern "C" {

int tans_encode_begin(const uint8_t* symbols, int64_t K, int64_t S, const int32_t* freqs,
                      int32_t nsym, const int32_t* spread, int32_t log2L, void** handle,
                      int64_t* comp_bytes, int64_t* n_offsets) {
    return encode_begin(symbols, K, S, freqs, nsym, spread, log2L, false, handle, comp_bytes,
                        n_offsets);
}

int tans_encode_packed_begin(const uint8_t* symbols, int64_t K, int64_t S, const int32_t* freqs,
                             int32_t nsym, const int32_t* spread, int32_t log2L, void** handle,
                             int64_t* comp_bytes, int64_t* n_offsets) {
    return encode_begin(symbols, K, S, freqs, nsym, spread, log2L, true, handle, comp_bytes,
                        n_offsets);
}

int tans_encode_finish(void* handle, uint8_t* comp, uint16_t* states, int64_t* offsets) {
    EncodeHandle* h = static_cast<EncodeHandle*>(handle);
    if (!h || !comp || !offsets || (!states && h->K && !h->packed)) {
        delete h;
        return fail(TANS_EINVAL, "encode_finish: null argument");
    }
    int64_t cum = 0;
    for (int64_t g = 0; g < h->n_groups; g++) {
        offsets[g] = cum;
        cum += (int64_t)h->streams[(size_t)g].size();
    }
    offsets[h->n_groups] = cum;
    uint32_t* c32 = reinterpret_cast<uint32_t*>(comp);
    #pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < h->n_groups; g++) {
        const auto& st = h->streams[(size_t)g];
        if (!st.empty()) std::memcpy(c32 + offsets[g], st.data(), st.size() * 4);
    }
    std::memset(c32 + cum, 0, (size_t)kTailWords * 4);
    if (h->K && !h->packed) std::memcpy(states, h->states.data(), (size_t)h->K * 2);
    delete h;
    return TANS_OK;
}

void tans_encode_free(void* handle) { delete static_cast<EncodeHandle*>(handle); }

}  // extern "C"
