/*
 * tans_amd.h -- C ABI of the MI355X (gfx950) fused tANS FP8 library.
 *
 * One shared library, libtans_amd.so, holds the CPU encoder and the HIP
 * kernels.  Every entry point takes plain pointers and sizes; device
 * pointers are HIP device memory, `stream` is a hipStream_t (NULL = the
 * null stream).  Launches are asynchronous on `stream`; the return code
 * covers argument validation and the launch itself.  All functions return
 * TANS_OK (0) or a negative TANS_E* code; tans_last_error() gives a message
 * for the calling thread's last failure.  Device buffers read or written
 * with vector loads must be aligned: FP8 inputs/outputs of the raw kernels,
 * compressed streams and the fused output 16 bytes, sign/mantissa tiles,
 * offsets and tables 8 bytes (TANS_EINVAL otherwise).
 *
 * Data format ("wave64 lane layout"):
 *   - The input is K lanes (rows) of N FP8 E4M3FN bytes.  A lane is one tANS
 *     state sequence; 64 consecutive lanes form a group, decoded by one
 *     wave64 (lane j of the group = wave lane j).
 *   - Symbols: the exponent nibble e = (b >> 3) & 15.  Pair alphabet: one
 *     symbol e0*16+e1 per two elements, table of 2^12 states.  Nibble
 *     alphabet: one symbol per element, 2^11 states, every present
 *     symbol's frequency at least 2.  The table size fixes the alphabet.
 *   - Bitstream: each lane's bits, in decode order, are cut into u32 words
 *     read LSB first; every decode step reads nb bits as one value.  The
 *     words of the 64 lanes of group g form one stream at
 *     comp_words[offsets[g] ..], ordered by the refill schedule all decoders
 *     follow: every active lane starts with two words (the stream's first
 *     words go to lanes 0, 1, ... in turn, then their second words).  The
 *     steps are cut into segments: step pairs (2p, 2p + 1) with 2^12-state
 *     tables; with 2^11-state tables, steps 8s .. 8s + 2, 8s + 3 .. 8s + 5
 *     and 8s + 6, 8s + 7 of every 8 (such tables give every present symbol
 *     a frequency of at least 2, so no step reads more than 10 bits).
 *     After each segment except the last, each active lane holding at most
 *     32 unread bits takes the next stream word (lanes in ascending order)
 *     and gains 32 bits; after the second-to-last segment only a lane
 *     holding fewer bits than the last segment can read does (24 with
 *     2^12-state tables, 10 per step of the last segment with 2^11),
 *     except when the last 16-element tile holds the last segment alone
 *     (N > 16 and N % 16 in 1..4 with 2^12-state tables, 1..3 with 2^11):
 *     that check is then the plain one.
 *     Streams start on 16-byte boundaries; 1 KiB of zero words follows the
 *     last one.  offsets is int64 [n_groups + 1], in words.
 *   - states[k] is lane k's initial decoder state in [L, 2L).
 *   - Packed layout of short streams (pair alphabet, N <= 64, written by
 *     tans_encode_packed_begin; a decoder is told by states == NULL): no
 *     state array and no refill schedule.  Group g's stream at
 *     comp_words[offsets[g] ..] is a header of 32 lane-pair bit counts
 *     (u8 when N <= 16, else u16, little-endian) and a bit area after it
 *     (bit b = bit b % 8 of its byte b / 8).  Pair p (lanes 2p, 2p + 1)
 *     owns bits [S_p, E_p): S_p = the counts of pairs 0 .. p - 1 summed,
 *     E_p = S_p + count p.  A lane's bits in decode order are (state - L)
 *     in 12 bits, then each step's nb bits, each value LSB first; the even
 *     lane's i-th bit is at S_p + i, the odd lane's at E_p - 1 - i.
 *     Lanes past K count 0 bits.  Streams start on 16-byte boundaries.
 *   - Sign/mantissa nibbles: 16-element tiles, 8 bytes per (tile, lane) at
 *     sm[(t * K + k) * 8]; u32 word h covers elements 8h..8h+7 as
 *     (A & 0x87878787) | rotl(B & 0x87878787, 4), A/B being elements
 *     8h..8h+3 / 8h+4..8h+7 read as little-endian words.
 *   - Decode table: L entries of two u32 words:
 *       word0 = nb | (e0 << 11) | (e1 << 19) | (nb << 27)
 *               (nibble alphabet: nb | (e << 11) | (nb << 27))
 *       word1 = (base - L) * 8
 *     for the state x = L + slot, with x_prev = f_sym + rank,
 *     nb = doublings of x_prev until >= L, base = x_prev << nb.
 */
#ifndef TANS_AMD_H
#define TANS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TANS_OK = 0,
    TANS_EINVAL = -1,     /* bad argument (shape, size, null pointer)      */
    TANS_ENOMEM = -2,     /* host allocation failed                          */
    TANS_ESYMBOL = -3,    /* a symbol outside the alphabet or of frequency 0  */
    TANS_ETABLE = -4,     /* freqs / spread inconsistent                     */
    TANS_EHIP = -5        /* a HIP runtime call failed                       */
};

#define TANS_LANES 64          /* lanes per group (one wave64)             */
#define TANS_TILE 16           /* elements per lane per tile                */
#define TANS_PAIR_LOG2L 12     /* table size of the pair alphabet          */
#define TANS_NIBBLE_LOG2L 11   /* table size of the nibble alphabet        */

/* Message for the calling thread's last failure ("" if none). */
const char* tans_last_error(void);

/* ---------------- CPU side ------------------------------------------- */

/* Split FP8 bytes into tANS symbols and packed sign/mantissa nibbles.
 * Replaces the nibble split / pair forming / sm packing of
 * rans_vectoradd/tans_codec.py:109-124.
 *   fp8      [K, N] bytes, N even
 *   sps      2 = pair alphabet (symbols [K, N/2]), 1 = nibble ([K, N])
 *   symbols  output, K*N/2 bytes (pair) or K*N bytes (nibble)
 *   sm       output, ceil(N/16) * K * 8 bytes (layout above)            */
int tans_split_fp8(const uint8_t* fp8, int64_t K, int64_t N, int32_t sps,
                   uint8_t* symbols, uint8_t* sm);

/* Host decode table from (spread, freqs).  Replaces
 * rans_vectoradd/tans_codec.py:63-87 and csrc/tans_decode.cu:23-59.
 *   spread [2^log2L] slot -> symbol; freqs [nsym], nsym 256 (pair, log2L
 *   12) or 16 (nibble, log2L 11); table output [2^log2L * 2] u32.       */
int tans_build_decode_table(const int32_t* spread, const int32_t* freqs,
                            int32_t nsym, int32_t log2L, uint32_t* table);

/* CPU encoder into the wave64 lane layout.  Together these replace
 * tans_encode_interleaved, csrc/tans_codec.cpp:69-196.
 * begin: encodes symbols [K, S] (S symbols per lane) with the table given
 *   by freqs [nsym] (summing to 2^log2L) and spread [2^log2L]; reports the
 *   output sizes.  finish: writes comp [comp_bytes], states [K] and
 *   offsets [n_offsets] and releases the handle.  free: releases a handle
 *   without writing (after an error).                                   */
int tans_encode_begin(const uint8_t* symbols, int64_t K, int64_t S,
                      const int32_t* freqs, int32_t nsym, const int32_t* spread,
                      int32_t log2L, void** handle, int64_t* comp_bytes,
                      int64_t* n_offsets);
int tans_encode_finish(void* handle, uint8_t* comp, uint16_t* states,
                       int64_t* offsets);
void tans_encode_free(void* handle);

/* tans_encode_begin into the packed layout of short streams (above):
 * 2^12-state tables (the pair alphabet), 1 <= S <= 32 steps per lane.
 * Same handle: tans_encode_finish writes comp and offsets and leaves
 * states alone (it may be NULL; the layout has no state array).  Also
 * replaces tans_encode_interleaved, csrc/tans_codec.cpp:69-196, for lanes
 * of up to 64 FP8 bytes; the reference keeps one u16 state per stream
 * (tans_codec.cpp:122-124) and pads each stream to whole u32 slabs.     */
int tans_encode_packed_begin(const uint8_t* symbols, int64_t K, int64_t S,
                             const int32_t* freqs, int32_t nsym, const int32_t* spread,
                             int32_t log2L, void** handle, int64_t* comp_bytes,
                             int64_t* n_offsets);

/* Encode tables of (spread, freqs) for the GPU encoder: enc_tab [nsym] =
 * f_s | start_s << 16 (start_s = f_0 + ... + f_{s-1}), enc_next [2^log2L]
 * = L + slot of the rank-th occurrence of s at index start_s + rank.  The
 * tables the CPU encoder builds internally (tans_encode_begin).          */
int tans_build_encode_table(const int32_t* spread, const int32_t* freqs, int32_t nsym,
                            int32_t log2L, uint32_t* enc_tab, uint16_t* enc_next);

/* ---------------- GPU side (gfx950) ---------------------------------- */

/* C = A, 16-byte vectors; n % 16 == 0.  Replaces fp8_memcpy,
 * csrc/fp8_memcpy.cu:45-64 (the HBM-ceiling kernel).                   */
int tans_fp8_memcpy(const void* a, void* c, int64_t n, void* stream);

/* C[i] = fp8_e4m3(float(A[i]) + float(B[i])), round-to-nearest-even with
 * saturation to +-448; n % 16 == 0.  Replaces fp8_vecadd_raw,
 * csrc/vecadd.cu:268-288.                                              */
int tans_fp8_vecadd_raw(const void* a, const void* b, void* c, int64_t n,
                        void* stream);

/* Bandwidth probes at tans_fp8_vecadd_raw's launch shape with the arithmetic
 * taken out; no counterpart in the reference, whose fp8_memcpy
 * (csrc/fp8_memcpy.cu:45-64, "practical bandwidth ceiling" at :71-73) is
 * the one ceiling it measures.  mode 0 reads A (n bytes), mode 1 writes C,
 * mode 2 writes C = A xor B (the raw add's two reads per write).
 * nontemporal != 0 uses non-temporal loads and stores (the raw add's
 * policy).  Mode 0 may store 4 bytes to sink.  n % 16 == 0; buffers a mode
 * does not use may be NULL.                                             */
int tans_stream_probe(int32_t mode, int32_t nontemporal, const void* a, const void* b,
                      void* c, int64_t n, void* sink, void* stream);

/* Device decode table from device spread/freqs (no host round trip):
 * the build of rans_vectoradd/tans_codec.py:63-87 and csrc/tans_decode.cu:23-59,
 * same output as tans_build_decode_table.  The kernel checks what the host
 * builder checks (frequencies summing to 2^log2L, every present symbol of a
 * 2^11-state table at frequency >= 2, spread symbols in the alphabet, slot
 * counts equal to frequencies) and, on a failure, sets *status (a device
 * int, may be NULL; the caller zeroes it) to TANS_ETABLE, in stream order.
 * A failed table still decodes without out-of-range accesses, to wrong
 * bytes.                                                                */
int tans_build_decode_table_device(const int32_t* spread, const int32_t* freqs,
                                   int32_t nsym, int32_t log2L, uint32_t* table,
                                   int32_t* status, void* stream);

/* Fused decode of two encodings (same table) + FP8 add.
 * out is tiled [N/16, K, 16]: out[(t*K + k)*16 + i] = element 16t+i of
 * lane k.  N % 16 == 0.  comp_bytes_* bound the reads: malformed offsets
 * cannot make a kernel read outside the buffers.  a_states and b_states
 * both NULL: both encodings are in the packed layout (log2L 12, N <= 64).
 * Replaces fp8_vecadd_fused_tans, csrc/vecadd.cu:290-393.               */
int tans_fp8_vecadd_fused(const void* a_comp, int64_t a_comp_bytes,
                          const int64_t* a_offsets, const uint16_t* a_states,
                          const void* a_sm,
                          const void* b_comp, int64_t b_comp_bytes,
                          const int64_t* b_offsets, const uint16_t* b_states,
                          const void* b_sm,
                          const uint32_t* table, int32_t log2L,
                          int64_t K, int64_t N, void* out, void* stream);

/* Standalone decode to FP8 bytes, out [N, K] (element-major, lane-minor).
 * N even.  states NULL: the packed layout (log2L 12, N <= 64).  Replaces
 * gpu_tans_decode, csrc/tans_decode.cu:159-210.                         */
int tans_decode(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                const uint16_t* states, const void* sm,
                const uint32_t* table, int32_t log2L,
                int64_t K, int64_t N, void* out, void* stream);

/* GPU encoder: the same bytes as tans_encode_begin/finish + tans_split_fp8
 * (the reference's tans_encode_interleaved, csrc/tans_codec.cpp:69-196, and
 * the split of rans_vectoradd/tans_codec.py:109-124), from FP8 bytes already
 * on the device.  Three calls:
 *   workspace  bytes of device scratch begin and finish need for [K, N]
 *   begin      fp8 [K, N] (device, 16-byte aligned, N even), enc_tab/enc_next from
 *              tans_build_encode_table (device copies), log2L 12 (pair) or
 *              11 (nibble).  Writes offsets [ceil(K/64) + 1] (int64 words),
 *              states [K], sm tiles (layout above), and sets *status (device
 *              int, zero on entry) to TANS_ESYMBOL if a symbol has frequency
 *              0.  The caller reads offsets[ceil(K/64)] (the stream words)
 *              and *status after the stream has reached this point.
 *   finish     writes comp: offsets[last] stream words + 256 zero words;
 *              comp_bytes = (offsets[last] + 256) * 4.
 * The workspace must stay untouched between begin and finish.           */
int tans_gpu_encode_workspace(int64_t K, int64_t N, int32_t log2L, int64_t* workspace_bytes);
int tans_gpu_encode_begin(const void* fp8, int64_t K, int64_t N, const uint32_t* enc_tab,
                          const uint16_t* enc_next, int32_t log2L, void* workspace,
                          int64_t workspace_bytes, int64_t* offsets, uint16_t* states, void* sm,
                          int32_t* status, void* stream);
int tans_gpu_encode_finish(int64_t K, int64_t N, int32_t log2L, const void* workspace,
                           const int64_t* offsets, void* comp, int64_t comp_bytes, void* stream);

/* The GPU encoder into the packed layout of short streams (log2L 12, N <= 64):
 * the same bytes as tans_encode_packed_begin/finish, with the same
 * workspace, the same calls and no states output.  Replaces, like those,
 * tans_encode_interleaved (csrc/tans_codec.cpp:69-196) for lanes of up to
 * 64 FP8 bytes.                                                          */
int tans_gpu_encode_packed_begin(const void* fp8, int64_t K, int64_t N, const uint32_t* enc_tab,
                                 const uint16_t* enc_next, int32_t log2L, void* workspace,
                                 int64_t workspace_bytes, int64_t* offsets, void* sm,
                                 int32_t* status, void* stream);
int tans_gpu_encode_packed_finish(int64_t K, int64_t N, int32_t log2L, const void* workspace,
                                  const int64_t* offsets, void* comp, int64_t comp_bytes,
                                  void* stream);

/* ---------------- Fused decode + skinny GEMM (no counterpart in the
 * reference: its rows a15 / configs 3-4 are new) ----------------------- */

/* y[b][r] = bf16(scale * sum_c W[r][c] * x[b][c]), fp32 accumulation,
 * round-to-nearest-even to bf16; W is R x C FP8 E4M3FN, tANS-coded as
 * written by rans_vectoradd.tans_codec.encode_matrix: rows padded to
 * Rp = R rounded up to 64, columns cut into S segments of Nc columns (a
 * multiple of 32, <= 1024) with (S - 1) * Nc < C <= S * Nc.  Lane
 * ((s * Rp / 16 + g) * 4 + q) * 16 + r holds row 16 g + r of segment s:
 * of each 64-column block of the segment, columns 16 q .. 16 q + 15, and
 * of a last block of 32 columns, columns 8 q .. 8 q + 7 (padding bytes
 * are multiplied by zero).  comp/offsets/states/sm are that encoding
 * (K = 4 * S * Rp lanes of Nc / 4 elements) and table its decode table.
 *   x          bf16 [B, C], 1 <= B <= 8
 *   workspace  device memory of at least S * B * Rp * 4 bytes, 16-byte
 *              aligned (per-segment fp32 partial sums; contents on entry
 *              do not matter)
 *   y          bf16 [B, R]
 * Partial sums are added in a fixed order, so results are deterministic. */
int tans_fp8_gemm_fused(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                        const uint16_t* states, const void* sm, const uint32_t* table,
                        int32_t log2L, int64_t R, int64_t C, int64_t S, int64_t Nc,
                        const void* x, int64_t B, float scale, void* workspace,
                        int64_t workspace_bytes, void* y, void* stream);

/* tans_fp8_gemm_fused without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  The partial sums go to a 16 MiB
 * device array inside the library (one per GPU, held until the process
 * ends), so S * B * Rp * 4 must not exceed 16 MiB (config 4's 17408 x 5120
 * and 5120 x 17408 layers fit at B = 8); larger products return
 * TANS_EINVAL.  Every call on one GPU uses that GPU's array: calls that
 * overlap in time on one GPU (different streams, host threads) race on it
 * and must be ordered by the caller.  Otherwise the same arguments, checks
 * and results as tans_fp8_gemm_fused.                                     */
int tans_fp8_gemm_fused_noalloc(const void* comp, int64_t comp_bytes, const int64_t* offsets,
                                const uint16_t* states, const void* sm, const uint32_t* table,
                                int32_t log2L, int64_t R, int64_t C, int64_t S, int64_t Nc,
                                const void* x, int64_t B, float scale, void* y, void* stream);

/* The same product from uncompressed FP8 W [R, C] (row-major), C % 16 == 0:
 * the baseline the fused kernel is measured against.                    */
int tans_fp8_gemm_raw(const void* w, int64_t R, int64_t C, const void* x, int64_t B,
                      float scale, void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TANS_AMD_H */
