/*
 * libkvq — C ABI of the MI355X (gfx950) packed-KV decode hot path.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (hipMalloc / torch CUDA tensors) unless stated otherwise.
 *   - Sizes are int64 element counts; strides are in elements of the pointed-to type.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Launches are asynchronous:
 *     nothing here synchronises the device, allocates device memory or keeps state between
 *     calls, so every call is HIP-graph capturable.
 *   - Return value: KVQ_OK (0) on success; KVQ_EINVAL when an argument is rejected before
 *     any launch; KVQ_EHIP when the HIP runtime reported an error.  kvq_last_error() returns
 *     the message of the last failure on the calling thread.
 *   - fp16 metadata (KIVI zero points `lo` and scales) is passed as raw uint16 bit patterns.
 *
 * The reference (TahirSher/KV-Project) is Python; its "FFI" for this path is the set of
 * Python functions each entry point replaces, cited per declaration as FILE:LINE.
 */
#ifndef KVQ_H_
#define KVQ_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVQ_OK 0
#define KVQ_EINVAL 1
#define KVQ_EHIP 2

/* element type codes */
#define KVQ_F32 0
#define KVQ_F16 1
#define KVQ_BF16 2

/* Message of the last failed call on this thread ("" if none). */
const char* kvq_last_error(void);

/* ABI version of the library (bumped on any signature change). */
int kvq_abi_version(void);

/* ------------------------------------------------------------------------------------------
 * A1  KIVI group quantisation (+ fused MSB-first packing).
 * Replaces kivi_quant (STRATA_KV.py:826-856) and, for the packed output, pack_codes applied to
 * its codes (STRATA_KV.py:2728-2732, as payload_bytes uses it, 2752-2755).
 *
 * x: (B, H, T, d) of x_dtype with element strides (sb, sh, st); channels contiguous.
 * Rows [0, n_sink) are not quantised.  n = T - n_sink rows are.
 * along_tokens != 0 (keys): per channel over groups of `group` tokens; n_g = ceil(n / group);
 *     lo, scale: (B, H, n_g, d) fp16, (b,h) stride meta_bh elements.
 * along_tokens == 0 (values): per token over groups of `group` channels (d when d % group);
 *     lo, scale: (B, H, n, d / width) fp16, (b,h) stride meta_bh elements.
 * codes  (optional, may be NULL): (B, H, n, d) uint8, (b,h) stride codes_bh bytes.
 * packed (optional): MSB-first packed codes of each (b,h) row block, rows of d*bits/8 bytes,
 *     (b,h) stride packed_bh bytes.  Requires bits in {2, 4, 8}.
 * xhat   (optional): (B, H, T, d) float32 contiguous = sinks exact + codes*scale+lo.
 * Bit-exact with the reference: fp16 round-to-nearest-even of lo and scale, IEEE fp32 division,
 * round-half-even codes, clamp to [0, 2^bits - 1], scale clamped at 2^-24.
 * ---------------------------------------------------------------------------------------- */
int kvq_kivi_quant(const void* x, int x_dtype, int64_t B, int64_t H, int64_t T, int64_t d,
                   int64_t sb, int64_t sh, int64_t st, int bits, int group, int along_tokens,
                   int n_sink, uint8_t* codes, int64_t codes_bh, uint8_t* packed,
                   int64_t packed_bh, uint16_t* lo, uint16_t* scale, int64_t meta_bh,
                   float* xhat, void* stream);

/* ------------------------------------------------------------------------------------------
 * A3  Bit packing.  kvq_pack_codes replaces pack_codes (STRATA_KV.py:2728-2732): `count`
 * uint8 codes (< 2^bits) -> ceil(count*bits/8) bytes, first code in the most significant bits,
 * last byte zero padded.  kvq_unpack_codes is its inverse.  bits in {1, 2, 4, 8}.
 * ---------------------------------------------------------------------------------------- */
int kvq_pack_codes(const uint8_t* codes, int64_t count, int bits, uint8_t* out, void* stream);
int kvq_unpack_codes(const uint8_t* packed, int64_t count, int bits, uint8_t* out, void* stream);
/* A3  Decode of pack_rows bytes (QUASAR_KV.py:1185-1190: per row, first code in the most
 * significant bits; for rows of whole bytes the same bytes as kvq_pack_codes row by row) through
 * the byte table of QUASAR_KV.py:1194-1202: out[i * 8/bits + s] = levels[code s of byte i].
 * levels: 2^bits float32 (device).  bits in {1, 2, 4, 8}. */
int kvq_unpack_rows_lut(const uint8_t* packed, int64_t n_bytes, int bits, const float* levels, float* out,
                        void* stream);

/* ------------------------------------------------------------------------------------------
 * A3  KIVI value-code decode layout (no reference counterpart: the reference never reads
 * packed KIVI bytes at decode; its stored format is pack_codes, STRATA_KV.py:2752-2755).
 * Value codes are kept in 32-token tiles laid out for the decode kernel's matrix-core operand
 * (each 32-bit word holds 8 tokens of one channel); per-token fp16 (scale, lo) pairs of every
 * channel group are kept per tile in the same token order.  These two calls convert between
 * pack_codes rows and the tile layout, both directions, bit-exact.
 *   rows:  (BH, n, d/2) bytes, (b,h) stride rows_bh; tiles: (BH, cap_t/32, 16*d) bytes,
 *   (b,h) stride cap_t*d/2.  Rows past n in the last tile are written as code 0.
 *   meta:  lo/scale (BH, n, ngv) fp16 -> vmeta (BH, cap_t/32, ngv, 32, 2) fp16.
 * Only 4-bit codes and d % 64 == 0 are supported.
 * ---------------------------------------------------------------------------------------- */
int kvq_v_tile(const uint8_t* rows, int64_t BH, int64_t n, int64_t rows_bh, int64_t d,
               int64_t cap_t, uint8_t* tiles, void* stream);
int kvq_v_untile(const uint8_t* tiles, int64_t BH, int64_t n, int64_t d, int64_t cap_t,
                 uint8_t* rows, int64_t rows_bh, void* stream);
int kvq_vmeta_tile(const uint16_t* lo, const uint16_t* scale, int64_t BH, int64_t n, int64_t ngv,
                   int64_t meta_bh, int64_t cap_t, uint16_t* vmeta, void* stream);

/* ------------------------------------------------------------------------------------------
 * A4  Split-K flash decoding over a packed 4-bit KIVI cache plus exact rows.
 * Replaces LayerState.attend -> chunked_attention over KIVI token entries
 * (STRATA_KV.py:716-719, 641-675, entries from 801-823) for a decode step.
 *
 * q: (B, Hq, Tq, d) of q_dtype, element strides (q_sb, q_sh, q_st), channels contiguous.
 *    KV head h serves query heads h*rep .. h*rep+rep-1 (STRATA_KV.py:527-529); the rows of
 *    KV head h are (query head, t) pairs, R = rep*Tq <= 8.
 * Packed cache of capacity cap_t tokens per (b,h), n_q tokens valid:
 *    kc    (B*Hkv, cap_t, d/2)  uint8, pack_codes rows (STRATA_KV.py:2728-2732)
 *    k_lo, k_sc (B*Hkv, cap_t/group_k, d) fp16
 *    vc    (B*Hkv, cap_t/32, 16*d) uint8 value tiles (kvq_v_tile)
 *    vmeta (B*Hkv, cap_t/32, d/group_v, 32, 2) fp16 (kvq_vmeta_tile)
 * Exact rows: k_exact, v_exact (B*Hkv, cap_e, d) of exact_dtype, 16-byte aligned, rows
 *    [0, n_exact) used.
 *    exact_pos (cap_e,) int64 and q_pos (Tq,) int64 (device, both may be NULL = every exact
 *    row visible): exact row i is visible to query t iff exact_pos[i] <= q_pos[t].
 *    Every packed row is visible to every query.
 * out: (B, Tq, Hq, d) of out_dtype, contiguous (the reference's output layout).
 * workspace: float32 scratch of kvq_kivi_decode_workspace(...) floats (split partials).  Calls
 *    sharing one workspace must not overlap in time (same stream, or ordered streams).
 * split_tokens: target packed tokens per workgroup (the packed rows of each (b,h) are cut into
 *    ceil(n_q / split_tokens) splits of equal 32-token chunk counts; 0 = automatic: the split
 *    count whose launch fills whole rounds of resident workgroups).
 * scores (optional, NULL = plain decode): (B*Hkv, scores_bh) float32, one row per (b, KV head)
 *    over the n_q packed positions.  The score pass adds score_weight * (sum over the rows of the
 *    KV head of each row's softmax probability of the packed token) to scores[bh][t]: the
 *    decode-time form of SnapKV's scores (STRATA_KV.py:932-954: mean over the query heads of a
 *    KV group and over queries, with score_weight = 1 / (rep * Tq * steps)).  The softmax runs over
 *    packed and visible exact rows, as the decode's.
 *    With a workspace of at least kvq_kivi_score_workspace(...) floats, a scored step's split
 *    kernel also spills its logits (fp32, into the workspace after the partials) and the scores
 *    come from them in one light pass; with kvq_kivi_decode_workspace(...) floats the score pass
 *    reads the keys again.  Both give the same scores bit for bit.
 * phases (bit mask): 1 = split kernel (partials of the packed splits and the exact rows into the
 *    workspace; with scores and a score workspace, the logits too); 2 = merge kernel (log-sum-exp
 *    merge, output write, and each row's global max/sum into the workspace); 4 = score pass (needs
 *    scores; reads the row statistics of a merge of the same call or an earlier one with the same
 *    args, and with a score workspace the logits of that call's phase 1).  3 = decode, 7 = decode
 *    + scores.
 * Requires d == 128, 4-bit codes, group_k % 32 == 0, group_v in {32, 64, 128}.
 * ---------------------------------------------------------------------------------------- */
int64_t kvq_kivi_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                                  int64_t n_q, int64_t n_exact, int group_k, int group_v,
                                  int64_t split_tokens);
/* Workspace floats of a scored step that spills its logits: kvq_kivi_decode_workspace's, rounded up
 * to 4, plus 32 * R floats per 32-token chunk and (b, h).  No reference counterpart of its own:
 * the scores it serves replace snapkv_scores (STRATA_KV.py:932-954) at decode time. */
int64_t kvq_kivi_score_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                                 int64_t n_q, int64_t n_exact, int group_k, int group_v,
                                 int64_t split_tokens);
int kvq_kivi_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling,
                    const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc,
                    const uint8_t* vc, const uint16_t* vmeta, int64_t cap_t, int64_t n_q,
                    int group_k, int group_v, const void* k_exact, const void* v_exact,
                    int exact_dtype, int64_t cap_e, int64_t n_exact, const int64_t* exact_pos,
                    const int64_t* q_pos, void* out, int out_dtype, float* workspace,
                    int64_t workspace_floats, float* scores, int64_t scores_bh, float score_weight,
                    int64_t split_tokens, int phases, void* stream);

/* ------------------------------------------------------------------------------------------
 * A4  kvq_kivi_decode without a workspace: the allocation-free variant.
 * No counterpart in the reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the caller
 * passes inputs and outputs only, and the call allocates nothing.
 *
 * Arguments and results as kvq_kivi_decode, minus (workspace, workspace_floats).  The split
 * partials and row statistics live in a static device array of KVQ_NOALLOC_SCRATCH_FLOATS
 * floats (8 MiB), one copy per GPU, held until the process ends; its device address is looked
 * up on the first call on each device.  The stream must belong to the current device.  A step
 * whose kvq_kivi_decode_workspace(...) exceeds KVQ_NOALLOC_SCRATCH_FLOATS is rejected
 * (KVQ_EINVAL) before any launch (C2, the 8B-shape layer at batch 16 and 32k tokens, needs
 * 400,384).  Nothing in the scratch has to start at zero: every partial and statistic the merge
 * and the score pass read is written earlier in the same call.  The scratch keeps the last
 * call's contents, and every call on a GPU shares it: calls that overlap in time on one GPU
 * (different streams without ordering) race and give wrong results.  Unlike every other entry
 * point, this one keeps state between calls (the scratch and its per-device address).
 * ---------------------------------------------------------------------------------------- */
#define KVQ_NOALLOC_SCRATCH_FLOATS (1 << 21)
int kvq_kivi_decode_noalloc(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling,
                            const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc,
                            const uint8_t* vc, const uint16_t* vmeta, int64_t cap_t, int64_t n_q,
                            int group_k, int group_v, const void* k_exact, const void* v_exact,
                            int exact_dtype, int64_t cap_e, int64_t n_exact, const int64_t* exact_pos,
                            const int64_t* q_pos, void* out, int out_dtype, float* scores,
                            int64_t scores_bh, float score_weight, int64_t split_tokens, int phases,
                            void* stream);

/* ------------------------------------------------------------------------------------------
 * A7  Top-k retention of accumulated scores.  Replaces scores.topk(k).indices.sort() of the
 * SnapKV / MTLP selection (STRATA_KV.py:975, 1022-1023): for each of BH rows of n float32
 * scores (row stride scores_bh), writes the positions of the k largest in increasing order to
 * idx (int32, row stride idx_bh).  Among scores equal to the k-th largest the lowest positions
 * are kept (the reference's torch.topk leaves that order unspecified).  The caller keeps the
 * recent window (the exact rows) by passing only the packed positions.  0 <= k <= n < 2^31.
 * ---------------------------------------------------------------------------------------- */
int kvq_topk_retain(const float* scores, int64_t BH, int64_t n, int64_t scores_bh, int64_t k,
                    int32_t* idx, int64_t idx_bh, void* stream);

/* The same selection (same result, bit for bit) spread over several workgroups per row, for
 * 4096 < n <= 2^24 and BH <= 65535: slices of 4096 scores, a row histogram, a candidate list and
 * per-slice output offsets kept in a caller's workspace of kvq_topk_retain_workspace(BH, n) 32-bit
 * words (256-byte aligned; contents need no clearing; calls sharing it must not overlap in time).
 * kvq_topk_retain_workspace returns 0 outside that range, and kvq_topk_retain_ws then runs
 * kvq_topk_retain (the workspace is not used).  Same replaced call as kvq_topk_retain
 * (STRATA_KV.py:975, 1022-1023). */
int64_t kvq_topk_retain_workspace(int64_t BH, int64_t n);
int kvq_topk_retain_ws(const float* scores, int64_t BH, int64_t n, int64_t scores_bh, int64_t k,
                       int32_t* idx, int64_t idx_bh, uint32_t* workspace, int64_t workspace_words,
                       void* stream);

/* ------------------------------------------------------------------------------------------
 * A7  SnapKV scores of a prefilled context.  Replaces snapkv_scores (STRATA_KV.py:932-954), the
 * selection of SnapKVMethod.entries (969-981) and of MTLP (1010-1023).
 *
 * q: the `window` observation queries of every query head, element (b, head, i, c) at
 *    q + b*q_sb + head*q_sh + i*q_st + c (query i at position H - window + i; the caller passes the
 *    view q[:, :, H - window:H]); k: (b, h, j, c) at k + b*k_sb + h*k_sh + j*k_st + c, j < H.  Both
 *    of `dtype`, channels contiguous, rows 16-byte aligned, d = 128; KV head h serves query heads
 *    h*rep .. h*rep + rep - 1 (STRATA_KV.py:527-529).
 * out (B*Hkv, H) float32: for j < H - window, the probability of key j under the causal fp32 softmax
 *    of scaling * q.k, averaged over the window queries and the rep heads, then avg_pool1d(kernel,
 *    padding kernel / 2, zeros counted); columns j >= H - window get (largest score of the whole
 *    call) + 1.  kernel odd, at most 65.  workspace: kvq_snapkv_scores_workspace(...) floats.
 * ---------------------------------------------------------------------------------------- */
int64_t kvq_snapkv_scores_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t window, int64_t H, int dtype);
int kvq_snapkv_scores(const void* q, int dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k,
                      int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t B, int64_t Hq, int64_t Hkv, int64_t d,
                      int64_t window, int64_t H, float scaling, int kernel, float* out, float* workspace,
                      int64_t workspace_floats, void* stream);

/* ------------------------------------------------------------------------------------------
 * F1  STRATA coverage statistics: replaces coverage_stats, STRATA_KV.py:1225-1298 (the groups of
 * coverage_groups 1206-1222 are drawn by the host, as the reference draws them, and passed as a plan).
 *
 * Plan (host-built, int32, device memory): G kept groups (those reaching the coded range); group g
 *    owns rows [row_base, row_base + rep*nq_pad) of every KV head, laid out [query head r][query i <
 *    nq_pad] (nq_pad = nq rounded up to 16).  gtab (G, 8): row_base, nq, nq_pad, mmax (max position
 *    + 1), te = min(re, mmax), local (1 for the window group, STRATA_LOCAL otherwise), 0, 0.
 *    rowpos (NR): the position of each row, -1 for padding; rowgrp (NR): its group; rlist (rep,
 *    n_rlist): the rows of query head r (-1 for padding); items (n_items, 2): (group, 64-row block)
 *    for every 64-row block of every group.  NR a multiple of 16.
 * qr: (Hkv, NR, d) of `dtype`, contiguous: row (h, row) = q[0, h*rep + r, position] (unscaled).
 * k, v: (h, j, c) at k + h*k_sh + j*k_st + c, j < T (batch element 0, as the reference), 16-byte
 *    aligned rows; M (Hq, d, d) float32: the output metric of each query head.  d = 128.
 * Outputs float32: A, W, DD (Hkv, re - rs); S, Mbar (Hkv, d, d) -- the reference's A, W, DD, S and
 *    Mbar with floor eta (STRATA_FLOOR).  workspace: kvq_coverage_stats_workspace(...) floats.
 *    Eleven launches on `stream`, no host synchronisation, deterministic (no atomics).
 * ---------------------------------------------------------------------------------------- */
int64_t kvq_coverage_stats_workspace(int64_t Hkv, int64_t rep, int64_t n, int64_t NR, int64_t G);
int kvq_coverage_stats(const void* qr, int dtype, int64_t NR, const int32_t* rowpos, const int32_t* rowgrp,
                       const int32_t* rlist, int64_t n_rlist, const int32_t* gtab, int64_t G, const int32_t* items,
                       int64_t n_items, const void* k, int64_t k_sh, int64_t k_st, const void* v, int64_t v_sh,
                       int64_t v_st, int64_t T, const float* M, int64_t Hkv, int64_t rep, int64_t d, int64_t rs,
                       int64_t re, float scaling, float eta, float* A, float* W, float* DD, float* S, float* Mbar,
                       float* workspace, int64_t workspace_floats, void* stream);

/* ------------------------------------------------------------------------------------------
 * A7  Retained-set rows for the gathered decode.  For each (b, h) and i < count, position
 * t = idx[bh*idx_bh + i] of the packed cache (layout as kvq_kivi_decode) is dequantised the way
 * kivi_quant's xhat is (code * scale + lo in fp32, STRATA_KV.py:855) and written, rounded to
 * out_dtype, to k_out / v_out (B*Hkv, out_bh elements per (b,h), row i at i*d).  Positions must
 * lie in [0, n_valid); others produce NaN rows.  The decode over the retained set is then
 * kvq_kivi_decode with these rows (plus the recent window) as exact rows and n_q = 0.  d = 128;
 * k_out, v_out, k_lo and k_sc 16-byte aligned; out_bh a multiple of 8 (so a caller can write
 * the rows straight into a larger buffer that also holds the window).
 * ---------------------------------------------------------------------------------------- */
/* Decode over the retained set straight from the packed cache (the gather and the exact-row decode
 * fused): attention of q over the packed positions idx[bh][0..n_ret) (idx_bh stride; each row read
 * and dequantised in registers, code * scale + lo in fp32 as kivi_quant's xhat, STRATA_KV.py:855;
 * a position outside [0, n_q) counts as a masked row) and the n_exact exact rows (the window, with
 * the exact_pos / q_pos rule of kvq_kivi_decode) -- the LayerState.attend over an MTLP / SnapKV
 * selection of a KIVI cache (STRATA_KV.py:682-719, 1010-1033) without writing the kept rows out.
 * Cache fields as kvq_kivi_decode; key metadata 16-byte aligned.  workspace >=
 * kvq_kivi_retained_workspace(...) floats; one retained/exact-row launch plus the merge. */
int64_t kvq_kivi_retained_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t n_ret,
                                    int64_t n_exact);
int kvq_kivi_decode_retained(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B,
                             int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, float scaling, const uint8_t* kc,
                             const uint16_t* k_lo, const uint16_t* k_sc, const uint8_t* vc, const uint16_t* vmeta,
                             int64_t cap_t, int64_t n_q, int group_k, int group_v, const int32_t* idx, int64_t n_ret,
                             int64_t idx_bh, const void* k_exact, const void* v_exact, int exact_dtype,
                             int64_t cap_e, int64_t n_exact, const int64_t* exact_pos, const int64_t* q_pos,
                             void* out, int out_dtype, float* workspace, int64_t workspace_floats, void* stream);

int kvq_kivi_gather_dequant(const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc,
                            const uint8_t* vc, const uint16_t* vmeta, int64_t cap_t, int64_t n_valid,
                            int group_k, int group_v, int64_t BH, int64_t d, const int32_t* idx,
                            int64_t count, int64_t idx_bh, void* k_out, void* v_out, int out_dtype,
                            int64_t out_bh, void* stream);

/* ------------------------------------------------------------------------------------------
 * A3  Planar packing.  kvq_pack_planar replaces pack_planar (STRATA_KV.py:1171-1182): `rows`
 * rows of d uint8 codes (< 2^bits) -> rows of d*bits/8 bytes, byte i holding coordinate
 * p*d/P + i in bits [p*bits, (p+1)*bits), P = 8/bits.  kvq_unpack_planar is unpack_planar
 * (1185-1189).  bits in {2, 4, 8}.
 * ---------------------------------------------------------------------------------------- */
int kvq_pack_planar(const uint8_t* codes, int64_t rows, int64_t d, int bits, uint8_t* out, void* stream);
int kvq_unpack_planar(const uint8_t* packed, int64_t rows, int64_t d, int bits, uint8_t* codes, void* stream);

/* ------------------------------------------------------------------------------------------
 * A5  STRATA codec.  One side (keys or values) of a layer's coded tokens, as compress_layer does
 * it (STRATA_KV.py:1546-1548) with rotation_matrix (1110-1128) and strata_quantize (1158-1168):
 *   kvq_strata_center_rotate: x (BH, n, d) of x_dtype, (b,h) stride x_bh elements ->
 *     mu (BH, d) fp16 = fp16(mean over the n tokens), y (BH, n, d) float32 = (x - mu) R^T with
 *     R = H_d diag(signs) / sqrt(d) (signs: d float32 +-1 on the device).
 *   kvq_strata_quantize: rows idx[bh][0..m) of y (all n rows in order when idx is NULL) ->
 *     planar codes (BH, m, d*bits/8) and fp16 scales (BH, m): s = max(fp16(step * rms(y)), 2^-24),
 *     code = clamp(round(y / s + (2^bits - 1) / 2)); step = uniform_step(bits) (1132-1155).
 * The arithmetic order is fixed (float64 sums, fast Walsh-Hadamard transform with stages
 * h = 1 .. d/2 then * float32(1/sqrt(d))), so results are reproducible bit for bit; they equal the
 * reference's torch float32 results up to float32 rounding of mu, y and rms.  d == 128.
 * ---------------------------------------------------------------------------------------- */
int kvq_strata_center_rotate(const void* x, int x_dtype, int64_t BH, int64_t n, int64_t d, int64_t x_bh,
                             const float* signs, uint16_t* mu, float* y, void* stream);
int kvq_strata_quantize(const float* y, int64_t BH, int64_t n, int64_t d, const int32_t* idx, int64_t m,
                        int bits, float step, uint8_t* codes, uint16_t* scales, void* stream);

/* ------------------------------------------------------------------------------------------
 * A6 layout (no reference counterpart: the reference's Triton kernel reads planar rows).  Value
 * codes of a stratum in the STRATA decode kernel's tile layout: planar rows (BH, n, d*bits/8),
 * (b,h) stride rows_bh bytes -> tiles (BH, cap_t/32, 512*bits bytes), and fp16 value scales vs
 * (BH, n), stride vs_bh -> vsl (BH, cap_t/32, 32) in the kernel's token-slot order.  Positions
 * >= n hold code 0 / scale 0.  cap_t % 32 == 0, d == 128.
 * ---------------------------------------------------------------------------------------- */
int kvq_strata_v_tile(const uint8_t* rows, int64_t BH, int64_t n, int64_t rows_bh, int bits, int64_t cap_t,
                      uint8_t* tiles, const uint16_t* vs, int64_t vs_bh, uint16_t* vsl, void* stream);

/* ------------------------------------------------------------------------------------------
 * A6  STRATA decode.  Replaces StrataState.attend (STRATA_KV.py:1762-1795) with its strata read
 * by strata_tier_kernel (1450-1469; tier_reference 1751-1760) for a decode step, batch B >= 1.
 * q: (B, Hq, Tq, d) of q_dtype, strides as kvq_kivi_decode; R = rep*Tq <= 8; d == 128.
 * signs (d) float32 +-1 and mu_k, mu_v (B*Hkv, d) fp16: the rotation and means of the coded tokens.
 * Tier t (host arrays of n_tiers <= 16 entries): tier_bits[t] in {2,4,8}, tier_n[t] tokens, key
 *   planar rows tier_kc[t] (B*Hkv, n, d*bits/8), key scales tier_ks[t] (B*Hkv, cap) fp16 (zero
 *   past n), value tiles
 *   tier_vt[t] and slot-ordered value scales tier_vsl[t] of capacity tier_cap[t] (kvq_strata_v_tile).
 * Exact rows as kvq_kivi_decode (k_exact, v_exact (B*Hkv, cap_e, d) of q_dtype, exact_pos / q_pos).
 * out: (B, Tq, Hq, d) of q_dtype.  workspace: kvq_strata_decode_workspace(...) floats.
 * Logit of a coded token (base e in the reference, base 2 here with log2(e) folded in):
 *   s_j = ks_j (q^ . c_j) - ks_j (2^b - 1)/2 sum(q^) + scaling q . mu_K,   q^ = scaling q R^T;
 * output = [w_e o_exact + (sum_t w_t acc_t) R + (sum_t w_t l_t) mu_V] / (sum of all w l).
 * ---------------------------------------------------------------------------------------- */
int64_t kvq_strata_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t n_exact,
                                    int n_tiers, const int* tier_bits, const int64_t* tier_n);
int kvq_strata_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B, int64_t Hq,
                      int64_t Hkv, int64_t Tq, int64_t d, float scaling, const float* signs, const uint16_t* mu_k,
                      const uint16_t* mu_v, int n_tiers, const int* tier_bits, const int64_t* tier_n,
                      const int64_t* tier_cap, const uint8_t* const* tier_kc, const uint16_t* const* tier_ks,
                      const uint8_t* const* tier_vt, const uint16_t* const* tier_vsl, const void* k_exact,
                      const void* v_exact, int64_t cap_e, int64_t n_exact, const int64_t* exact_pos,
                      const int64_t* q_pos, void* out, float* workspace, int64_t workspace_floats, void* stream);

/* ------------------------------------------------------------------------------------------
 * A6  Flash-decoding partials of ONE stratum for a pre-rotated query.  Replaces the reference's
 * kernel wrapper strata_tier_kernel(qr, qb, t, target_programs) (STRATA_KV.py:1450-1469, the
 * Triton kernel 1374-1447), whose partials StrataState.attend merges (1782-1792).
 *
 * qr (BH, rows, d) float32 = scaling * q R^T (rotated, scaled query rows), qb (BH, rows) float32 =
 * scaling * q . mu_K.  The stratum: n tokens, kc (BH, n, d*bits/8) pack_planar rows, ks (BH, cap)
 * fp16 key scales zero past n, vt / vsl its value tiles and slot-ordered scales of capacity cap
 * (kvq_strata_v_tile).  The n tokens are cut into n_split splits (1 <= n_split <= ceil(n/32)).
 * Outputs, as the reference's: m, l, z (BH, n_split, rows) and acc (BH, n_split, rows, d) float32
 * in the rotated value basis, natural exponent: m = max logit, l = sum e^(s - m),
 * acc + z = sum e^(s - m) vs (c - (2^bits - 1)/2) (the offset is folded into acc; z = 0, as the
 * reference's tier_reference returns).  Any rows (launches of 8 rows).  d = 128.
 * ---------------------------------------------------------------------------------------- */
int kvq_strata_tier_partials(const float* qr, const float* qb, int64_t BH, int64_t rows, int64_t d, int bits,
                             int64_t n, const uint8_t* kc, const uint16_t* ks, const uint8_t* vt,
                             const uint16_t* vsl, int64_t cap, int64_t n_split, float* m, float* l, float* acc,
                             float* z, void* stream);

/* ------------------------------------------------------------------------------------------
 * C3  Mixed-width KIVI blocks.  Every 64-token block of a (b, h) has its own width b in
 * {2, 4, 8}; inside it the codes and fp16 metadata are kivi_quant's (STRATA_KV.py:826-856) at
 * that width with group 32.  The reference keeps one dense tensor per width and launches once per
 * width (StrataState.attend, STRATA_KV.py:1782-1783); here one flat buffer holds, per (b, h) from
 * 2 KiB unit bh_base[bh], the 8-bit blocks, then the 4-bit, then the 2-bit blocks (token order
 * within a width), a block of width b taking b + 1 units:
 *   0              key rows, planar (pack_planar, STRATA_KV.py:1171-1182), 64 x 16b bytes
 *   1024 b         value tiles of the two 32-token chunks (the STRATA tier tile layout), 512 b each
 *   2048 b         key scales sc[2][128] fp16, key zeros lo[2][128] fp16
 *   2048 b + 1024  value (scale | zero << 16) words per chunk [group 4][lane group 4][slot 8]
 * Offset table: blk_bits (BH, nb) and blk_off (BH, nb) int32 units from bh_base[bh].
 * kvq_mixed_encode: k, v (BH, nb*64, 128) of dtype, head stride x_bh; one workgroup per block.
 * kvq_mixed_decode: seg (BH, 4) int64 = (bh_base, n8, n4, n2); every block visible; exact rows
 * as kvq_kivi_decode's (dtype = q_dtype).  out (B, Tq, Hq, 128) of q_dtype.  phases: 1 = the
 * partials (exact rows and coded blocks) into the workspace, 2 = their merge into out, 3 = both.
 * ---------------------------------------------------------------------------------------- */
int kvq_mixed_encode(const void* k, const void* v, int dtype, int64_t BH, int64_t nb, int64_t d, int64_t x_bh,
                     const uint8_t* blk_bits, const int32_t* blk_off, const int64_t* bh_base, uint8_t* buf,
                     void* stream);
int64_t kvq_mixed_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t nb,
                                   int64_t n_exact);
int kvq_mixed_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t Tq, int64_t d, float scaling, const uint8_t* buf, const int64_t* seg,
                     int64_t nb, const void* k_exact, const void* v_exact, int64_t cap_e, int64_t n_exact,
                     const int64_t* exact_pos, const int64_t* q_pos, void* out, float* workspace,
                     int64_t workspace_floats, int phases, void* stream);

/* ------------------------------------------------------------------------------------------
 * A9  Blockwise token-axis DCT coding (no counterpart in the reference; the contract follows its
 * conventions: absmax_quant, STRATA_KV.py:549-554, and offset-binary 4-bit storage,
 * TILT_KV.py:2621-2625).  Per (b, h, 64-token block, channel): X_k = sum_n C[k][n] x_n for the
 * 16 kept rows of the orthonormal DCT-II, summed over n = 0..63 in increasing n in float32
 * without fused multiply-add; s = max(fp16(max|X| / 7), 2^-24); code = clamp(rint(X / s), -7, 7) + 7.
 * x: (BH, T, d) of x_dtype, row stride d, head stride x_bh; T % 64 == 0, d == 128.
 * ctab: (16, 64) float32 (float32 of the closed form).  Per block, 1024 code bytes and 128 fp16
 * scales: for_values == 0 -> key layout (16 rows of 16 32-bit words by coefficient: word D holds
 * channels 8D .. 8D+7, channel 8D + e at nibble {0,4,1,5,2,6,3,7}[e]; scales by channel);
 * for_values == 1 -> value tile (word (gp*16 + n)*8 + blk holds coefficients
 * 8gp .. 8gp+7 of channel 16*blk + n, coefficient 8gp + e at nibble {0,4,1,5,2,6,3,7}[e]; scales
 * ordered [n][blk]).
 * ---------------------------------------------------------------------------------------- */
int kvq_dct_encode(const void* x, int x_dtype, int64_t BH, int64_t T, int64_t d, int64_t x_bh,
                   const float* ctab, int for_values, uint8_t* codes, uint16_t* scales, void* stream);

/* Decode over a DCT-coded context of T tokens (T % 64 == 0, kc/ks key blocks, vc/vs value blocks,
 * each (B*Hkv, T/64, ...)) plus n_exact exact rows (as kvq_kivi_decode's exact rows, dtype =
 * q_dtype): attention over the reconstructions x_n = sum_k C[k][n] s_k (code_k - 7), computed in
 * the coefficient domain (logits C^T (K-codes q), values (V-codes) (C p)).  ctab: 2048 float32,
 * 16-byte aligned: the encoder's (16, 64) table followed by its transpose (64, 16).  out (B, Tq, Hq, d)
 * of q_dtype.  Workspace floats from kvq_dct_decode_workspace.  phases as kvq_mixed_decode's. */
int64_t kvq_dct_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t T,
                                 int64_t n_exact);
int kvq_dct_decode(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t B, int64_t Hq,
                   int64_t Hkv, int64_t Tq, int64_t d, float scaling, const float* ctab, int64_t T,
                   const uint8_t* kc, const uint16_t* ks, const uint8_t* vc, const uint16_t* vs,
                   const void* k_exact, const void* v_exact, int64_t cap_e, int64_t n_exact,
                   const int64_t* exact_pos, const int64_t* q_pos, void* out, float* workspace,
                   int64_t workspace_floats, int phases, void* stream);

/* ------------------------------------------------------------------------------------------
 * A2  Fused quantise + pack append of one token per sequence (streaming KIVI window).
 * No per-step quantiser exists in the reference (its decode-time appends stay exact,
 * STRATA_KV.py:707-714); this restates KIVIMethod's window rule (806-822) for a streaming cache:
 * a token is read exact while among the last W positions, then from its kivi_quant codes.
 * k_new, v_new: (B, Hkv, 1, d) of dtype with element strides (k_sb, k_sh) / (v_sb, v_sh).
 * k_ring, v_ring: (B*Hkv, W, d) of dtype, position p in slot p % W.  Packed cache as for
 * kvq_kivi_decode (capacity cap_t tokens).  For pos >= W, token pos-W is quantised (value row;
 * and, when (pos-W) % group_k == 0, key group (pos-W)/group_k from the ring) before the new row
 * is written into slot pos % W.  After the call the decode reads n_q = max(0, pos+1-W) packed
 * tokens and min(pos+1, W) ring rows.  Requires d == 128, 4-bit, W >= group_k, group_k % 32 == 0.
 * ---------------------------------------------------------------------------------------- */
int kvq_kivi_append(const void* k_new, const void* v_new, int dtype, int64_t k_sb, int64_t k_sh,
                    int64_t v_sb, int64_t v_sh, int64_t B, int64_t Hkv, int64_t d, int64_t pos,
                    void* k_ring, void* v_ring, int64_t W, uint8_t* kc, uint16_t* k_lo,
                    uint16_t* k_sc, uint8_t* vc, uint16_t* vmeta, int64_t cap_t, int group_k,
                    int group_v, void* stream);

/* ------------------------------------------------------------------------------------------
 * F4  Wire format and measured bytes of a packed KIVI layer: replaces payload_bytes
 * (STRATA_KV.py:2736-2769) for KIVI states, whose total must match the analytic state_bits
 * (773-783, entry_bits 798-799).  kvq_kivi_export writes, from the decode layout of
 * kvq_kivi_decode (same kc / k_lo / k_sc / vc / vmeta arguments), the sections
 *   key codes (pack_codes rows, n_q x d/2 bytes per bh), key lo, key scale (fp16, ceil(n_q /
 *   group_k) x d per bh), value codes (pack_codes rows), value lo, value scale (fp16, n_q x
 *   d/group_v per bh), exact keys, exact values (n_exact x d per bh as fp16, the reference's .half()
 *   of rows stored in exact_dtype; oldest first: slot (first_slot + i) % cap_e),
 * each (b, h)-major, into out (out_bytes >= kvq_kivi_payload_bytes(...)).  4-bit codes, d = 128.
 * ---------------------------------------------------------------------------------------- */
int64_t kvq_kivi_payload_bytes(int64_t BH, int64_t n_q, int64_t d, int group_k, int group_v, int64_t n_exact,
                               int exact_dtype);
int kvq_kivi_export(const uint8_t* kc, const uint16_t* k_lo, const uint16_t* k_sc, const uint8_t* vc,
                    const uint16_t* vmeta, int64_t BH, int64_t cap_t, int64_t n_q, int64_t d, int group_k,
                    int group_v, const void* k_exact, const void* v_exact, int exact_dtype, int64_t cap_e,
                    int64_t n_exact, int64_t first_slot, uint8_t* out, int64_t out_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * F2  QUASAR compressed-domain decode: replaces QuasarState.attend (QUASAR_KV.py:1945-1968) with
 * its coded part read from the packed bytes (the reference's _quasar_scores_kernel /
 * _quasar_values_kernel, 1498-1551, and their torch path, 1920-1943), batch 1.
 *   q (1, Hq, Tq, d = 128) of q_dtype, strides q_sh, q_st; exact rows k_exact / v_exact (1, Hkv,
 *   cap_e, d) of q_dtype, the first n_exact attended, row i visible to query t iff exact_pos[i] <=
 *   q_pos[t] when both are given (the causal rule of appended rows, 1950-1953).
 *   Per side (k_ / v_): codes (`bytes` long) = the steps' (Hkv, n_s, nb) pack_rows blocks, in step
 *   order, described by the side's step table, int32 rows [byte offset, n_s, nb, a, w, bits, level
 *   offset] (1883-1898; n_s non-increasing, nb in {4, 8, 16, 32, 64}, at most 128 bytes per token
 *   and side).  levels = the stage codebooks concatenated (float32, at most 256).  rho_k / rho_v
 *   (Hkv, n_c) fp16; T_k (Hkv, d, R_k) float32 and T_v transposed, (Hkv, R_v, d) fp16 (the
 *   precision the reference stores it at; R_k, R_v multiples of 4); mu_k / mu_v (Hkv, d) float32.  bounds (`splits` + 1 int32 chunk boundaries, 64-token chunks), slots (int32 [2][32][8])
 *   and the slot counts come from kvq_quasar_plan (device copies).  out (1, Tq, Hq, d) of
 *   q_dtype.  rep x Tq <= 8.  phases: mask of 1 (the
 *   query's coefficients), 2 (the split launch), 4 (the row merge, where up to 128 exact rows are
 *   attended); 7 for a decode step (the others are timing hooks that reuse the workspace of an
 *   earlier call).
 * kvq_quasar_plan: host-memory step tables in (checked); out, in host memory: chunk boundaries of
 * the splits, cut so that the longest split (its wavefronts claiming its chunks in order, chunk
 * costs from the coefficients the tokens own) is shortest within one resident round of workgroups
 * (bounds needs max_splits + 1 entries; *n_splits receives the split count) and the
 * slot table (2 x 32 x 8 int32: per 4-byte slot of a token's rows, the step offset + 4 dw, n_s, nb,
 * first coefficient, bits, level offset, step) with n_slots[2].  No reference counterpart (the
 * reference launches one program per 64-token block).
 * ---------------------------------------------------------------------------------------- */
int kvq_quasar_plan(const int32_t* k_table, int k_steps, const int32_t* v_table, int v_steps, int64_t n_c,
                    int64_t Hkv, int max_splits, int32_t* bounds, int32_t* n_splits, int32_t* slots,
                    int32_t* n_slots);
int64_t kvq_quasar_decode_workspace(int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d, int64_t R_k,
                                    int64_t n_exact, int splits);
int kvq_quasar_decode(const void* q, int q_dtype, int64_t q_sh, int64_t q_st, int64_t Hq, int64_t Hkv,
                      int64_t Tq, int64_t d, float scaling, const void* k_exact, const void* v_exact,
                      int64_t cap_e, int64_t n_exact, const int64_t* exact_pos, const int64_t* q_pos,
                      const uint8_t* k_codes, int64_t k_bytes, const uint8_t* v_codes, int64_t v_bytes,
                      const int32_t* slots, int nslots_k,
                      int nslots_v, const float* levels, int n_levels,
                      const uint16_t* rho_k, const uint16_t* rho_v, int64_t n_c, const float* T_k,
                      const uint16_t* T_v, int64_t R_k, int64_t R_v, const float* mu_k, const float* mu_v,
                      const int32_t* bounds, int splits, void* out, float* workspace,
                      int64_t workspace_floats, int phases, void* stream);

/* ------------------------------------------------------------------------------------------
 * F1  STRATA rate allocation of one layer (the compression side): replaces the allocation steps
 * of StrataMethod.compress_layer (STRATA_KV.py:1559-1581) -- nan_to_num of D, the per-head
 * importance order (1560), the head-summed table Dsort (1561), head_sync_allocate (1307-1351,
 * called at 1569), lev = choice sorted descending and its histogram (1570-1571), the distortion
 * ratio (1577-1581).
 *   D (Hkv, n, nlev) float32, columns [drop | level 1 .. level nlev-2 | exact]; cost (nlev) and
 *   fixed (nlev - 1) float64 HOST arrays (option bits summed over heads; fixed bits per cap);
 *   budget in bits; rounds of 32 multipliers (the reference's STRATA_ROUNDS), or rounds < 0 for
 *   the all-drop allocation (the reference's branch when the budget cannot pay the histogram).
 * Outputs (device): order (Hkv, n) int32, dsort (n, nlev) float32, choice (n) int32, lev (n)
 * int32, counts (nlev) int32, summary [bits, cap, distortion] float64.  The search runs in
 * float64 (products rounded before sums; drop wins ties against exact, the running minimum over
 * levels takes the later level, the cap is the first of minimal total); ties of the importance
 * key go to the lower token index.  workspace: 256-byte aligned, >= kvq_strata_allocate_workspace(...)
 *  bytes (-1: bad shape).  Hkv < 256, Hkv n < 2^31, 2 <= nlev <= 16.
 * ---------------------------------------------------------------------------------------- */
/* The distortion table the allocation reads, from the coverage statistics: replaces
 * compress_layer's metrics in the code basis (STRATA_KV.py:1543, R S R^T and R Mbar R^T), the
 * error term of each width on both sides (1546-1553: e = y_hat - y of strata_quantize, e^T Mt e)
 * and the table D = [DD | A errK_b + W errV_b per width | 0] (1555-1557).  yk / yv (Hkv, n, 128)
 * float32 are the centred, rotated coded rows (kvq_strata_center_rotate); S, Mbar (Hkv, 128, 128)
 * float32 in the original basis; signs the rotation signs; A, W, DD (Hkv, n) float32; bits /
 * steps (host, nbits <= 3 widths in {2, 4, 8} and their uniform_step); D (Hkv, n, nbits + 2)
 * float32 out.  workspace >= kvq_strata_distortion_workspace(...) bytes (-1: bad sizes). */
int64_t kvq_strata_distortion_workspace(int64_t Hkv, int64_t n, int nbits);
int kvq_strata_distortion(const float* yk, const float* yv, int64_t Hkv, int64_t n, int64_t d, const float* S,
                          const float* Mbar, const float* signs, const float* A, const float* W,
                          const float* DD, int nbits, const int* bits, const float* steps, float* D,
                          float* workspace, int64_t workspace_bytes, void* stream);

int64_t kvq_strata_allocate_workspace(int64_t Hkv, int64_t n, int nlev);
int kvq_strata_allocate(const float* D, int64_t Hkv, int64_t n, int nlev, const double* cost,
                        const double* fixed, double budget, int rounds, int32_t* order, float* dsort,
                        int32_t* choice, int32_t* lev, int32_t* counts, double* summary,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * A7  Eviction families that keep exact rows, and chunk-local selection.
 *
 * kvq_gather_rows: rows idx[bh][0..count) of one or two (b, h)-sliced row arrays (k, and v when
 * non-null; rows of row_bytes bytes, (b, h) stride x_bh bytes) into k_out / v_out (rows in idx
 * order, (b, h) stride out_bh bytes); an index outside [0, n_valid) writes a zero row.  It replaces
 * the torch.gather of the kept rows in SnapKVQuantMethod.entries (STRATA_KV.py:1024-1025) and the
 * column selection of LayerState.__init__ over a SnapKV / StreamingLLM keep set (682-694, hide
 * masks of 969-981 and 1048-1059).  row_bytes, strides and pointers multiples of 16 bytes.
 *
 * kvq_chunk_share: finalize_chunk's within-chunk attention share (STRATA_KV.py:581-583) --
 * share[bh][c] = (1/nq) sum_q softmax_c(qref[bh][q] . k[bh][c]) for qref (BH, nq, d) the scaled
 * observed queries and k (BH, C, d), both float32 and 16-byte aligned; C <= 2048, d % 4 == 0.
 * workspace >= kvq_chunk_share_workspace(BH, nq, C) floats (the logits).  The top-k of the share
 * (kvq_topk_retain) and the gather of the kept rows complete finalize_chunk's selection.
 *
 * kvq_absmax_fake_quant: fake_quant_tokens (STRATA_KV.py:556-563) for 2 <= bits <= 15 -- per row
 * of d float32, s = max(fp16(max|x| / qmax), 2^-24) with qmax = 2^(bits-1) - 1 and the value
 * saturated to the fp16 range, out = clamp(round_half_even(x / s), -qmax, qmax) * s (absmax_quant,
 * 549-554), bit-exact; out may alias x.
 * ---------------------------------------------------------------------------------------- */
int kvq_gather_rows(const void* k, const void* v, int64_t BH, int64_t n_valid, int64_t x_bh, int64_t row_bytes,
                    const int32_t* idx, int64_t count, int64_t idx_bh, void* k_out, void* v_out, int64_t out_bh,
                    void* stream);
int64_t kvq_chunk_share_workspace(int64_t BH, int64_t nq, int64_t C);
int kvq_chunk_share(const float* qref, const float* k, int64_t BH, int64_t nq, int64_t C, int64_t d, float* share,
                    float* workspace, int64_t workspace_floats, void* stream);
int kvq_absmax_fake_quant(const float* x, int64_t rows, int64_t d, int bits, float* out, void* stream);

/* ------------------------------------------------------------------------------------------
 * F2  QUASAR coded-domain products of one side, with the reference's kernel-wrapper call shapes
 * quasar_scores(qt, side, n_c) and quasar_values(pv, side, R) (QUASAR_KV.py:1556-1577).  A side
 * is QuasarState's stored code (1883-1898): the flat uint8 buffer (flat_bytes) of every step's
 * (Hkv, n_s, nb) pack_rows block, the step table -- n_steps <= 64 int32 rows [offset, n_s, nb, a,
 * w, bits, level offset], in HOST memory, checked against the buffers before any launch -- and the
 * concatenated stage codebooks levels (n_levels float32).
 *   kvq_quasar_scores: qt (Hkv, rows, R) float32 -> out (Hkv, rows, n_c) float32, out[h][r][j] =
 *     sum over the steps owning token j of qt[h][r][band] . levels[codes of j]   (n_c <= 65535 * 64)
 *   kvq_quasar_values: pv (Hkv, rows, n_c) float32 -> out (Hkv, rows, R) float32, out[h][r][c] =
 *     sum over the steps covering coefficient c and their tokens j of pv[h][r][j] levels[code];
 *     workspace >= kvq_quasar_values_workspace(...) floats.
 * Fixed summation order (steps, then band positions or tokens): reproducible bit for bit.
 * ---------------------------------------------------------------------------------------- */
int kvq_quasar_scores(const float* qt, int64_t Hkv, int64_t rows, int64_t R, const uint8_t* flat, int64_t flat_bytes,
                      const int32_t* table, int n_steps, const float* levels, int64_t n_levels, int64_t n_c,
                      float* out, void* stream);
int64_t kvq_quasar_values_workspace(int64_t Hkv, int64_t rows, int64_t R, int64_t n_c);
int kvq_quasar_values(const float* pv, int64_t Hkv, int64_t rows, int64_t n_c, const uint8_t* flat, int64_t flat_bytes,
                      const int32_t* table, int n_steps, const float* levels, int64_t n_levels, int64_t R,
                      float* out, float* workspace, int64_t workspace_floats, void* stream);

/* ------------------------------------------------------------------------------------------
 * Self-test of the matrix-core operand layout the decode kernel is written against
 * (v_mfma_f32_16x16x32_f16 on gfx950): writes, for A = I-pattern inputs, the 16x16 product
 * as each lane sees it, followed by the lane each lane reads under row_shr:4 and row_ror:4 and
 * the two results of v_permlane32_swap and v_permlane16_swap applied to the lane index.
 * a, b: 64*8 fp16 each (lane-major); out: 64*4 + 6*64 floats.  No reference counterpart
 * (layout check only).
 * ---------------------------------------------------------------------------------------- */
int kvq_selftest_mfma_layout(const uint16_t* a, const uint16_t* b, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KVQ_H_ */
