// Host-side launchers of the HIP kernels.  All pointers are device pointers;
// every launcher is asynchronous on `st` and returns hipSuccess or the launch error.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlg {

// A weight matrix W [N, K] resident in HBM.  Q4_K / Q5_K / F16 / F32 keep the
// GGUF bytes as they are; Q6_K and Q8_0 are split into planes at upload so that
// every plane is 16-byte aligned (same bytes in total, bit-identical dequant):
//   Q6_K: q = [N][nb][192] (ql | qh), s = [N][nb][16] int8 scales, d = [N][nb] f16
//   Q8_0: q = [N][K] int8,            d = [N][K/32] f16
struct DevMatrix {
    uint32_t type = 0;
    int N = 0, K = 0;
    uint8_t *q = nullptr, *s = nullptr, *d = nullptr;
    size_t bytes = 0;  // total bytes of the planes (= GGUF bytes)
    // q6_K LM heads: a second copy of the quant plane in lane-major order, read by the
    // large-matrix GEMVs (layout_lane_major); null elsewhere
    uint8_t *lm = nullptr;
    // q6_K / q4_K matrices: the MFMA GEMMs' copy in tile-major order (layout_tile_major);
    // null elsewhere
    uint8_t *tm = nullptr;
};

// Tile-major q6_K / q4_K (the MFMA GEMMs' W operand): per 16-row tile t < ceil(N / 16)
// and 256-wide K block kb, B bytes at (t * K/256 + kb) * B (rows past N are zero).  Lane
// l = 16 kq + r of a wave (row 16 t + r, k-group kq) finds what it multiplies in 16-byte
// pieces at 1024 j + 16 l, so every load of a wave reads whole cache lines:
//   q6_K (B = kQ6TileBytes): pieces j = 0: ql[64 n + 16 h + 4 kq], 1: ql[64 n + 32 + 16 h
//     + 4 kq], 2: qh[32 n + 16 h + 4 kq] (4 bytes each, dword 2 n + h of the piece); the
//     row's 16 scales at 3072 + 16 r and its f16 d at 3328 + 2 r;
//   q4_K (B = kQ4TileBytes): the row's 16-byte header (d, dmin, packed scales) at 16 r;
//     pieces at 256 + 1024 j + 16 l: qs[32 g + 8 kq .. + 8] for g = 2 j, 2 j + 1.
constexpr int kQ6TileBytes = 3456;
constexpr int kQ4TileBytes = 2304;
size_t tile_major_bytes(uint32_t type, int N, int K);  // 0: no tile-major form
// planes: q | s | d as layout_planes writes them (off_s, off_d: the plane offsets)
void layout_tile_major(uint32_t type, int N, int K, const uint8_t *planes, size_t off_s, size_t off_d,
                       uint8_t *out);

// Splits/copies GGUF rows [N][K] of `type` into the device layout (host side).
// Fills `host_planes` with q | s | d concatenated and the plane offsets.
bool layout_planes(uint32_t type, int N, int K, const uint8_t *gguf, uint8_t *out, size_t *off_s, size_t *off_d,
                   size_t *total);
size_t planes_bytes(uint32_t type, int N, int K);
// q6_K: the quant plane (block-major [N * K/256][192], as layout_planes writes it) in
// lane-major order: piece k of 64-value chunk c of row r (k = 0, 1: the two 16-byte ql
// pieces, 2: the 16-byte qh piece a GEMV lane reads) at k * N * (K/256) * 64 +
// (r * (K/64) + c) * 16.  The lanes of a row group then read whole cache lines per load.
size_t lane_major_bytes(uint32_t type, int N, int K);  // 0: no lane-major form
void layout_lane_major(int N, int K, const uint8_t *q_plane, uint8_t *out);

// Largest batch the register-resident GEMV handles for this matrix (0 if none).
int gemv_max_batch(const DevMatrix &w);
// Workgroups of a GEMV launch over w.
int gemv_grid(const DevMatrix &w, int G = 2);  // G: row groups per wave and step

// y[b][n] = sum_k x[b][k] W[n][k] (+ bias[n]) (relu if set).  b <= gemv_max_batch(w).
hipError_t gemv(const DevMatrix &w, const float *x, int ldx, int b, float *y, int ldy, const float *bias, bool relu,
                hipStream_t st);
// Same product, but each workgroup writes the argmax (ties -> lowest index) of its
// rows to pv/pi [b][parts]; logits are not stored.  Index `mask_id` (>= 0) is skipped.
// ln (optional, integer formats): the GEMV's x is LayerNorm(ln->x + ln->y) ([b][K] rows,
// residual_ln's arithmetic) computed inside the launch; ln->h (if set) receives it.
struct GemvLn {
    const float *x, *y, *g, *b;
    float eps;
    float *h;
};
hipError_t gemv_argmax(const DevMatrix &w, const float *x, int ldx, int b, int mask_id, float *pv, uint32_t *pi,
                       int *parts, hipStream_t st, const GemvLn *ln = nullptr);
// Number of partial results gemv_argmax writes per batch row.
int gemv_argmax_parts(const DevMatrix &w, int b);

// Y[m][n] = sum_k X[m][k] W[n][k] + bias[n] (+ R[m][n]) (relu if set); any M.
// Runs on the MFMA units when gemm_mfma_supported(w) (K % 256 == 0, quantized or
// f16 weights), else on the SIMT kernel.
// ws (optional, ws_bytes): workspace for split-K partial sums when M is small; the
// partials are added in a fixed order.
hipError_t gemm(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias, bool relu,
                const float *R, int ldr, hipStream_t st, float *ws = nullptr, size_t ws_bytes = 0);
hipError_t gemm_simt(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias,
                     bool relu, const float *R, int ldr, hipStream_t st);
bool gemm_mfma_supported(const DevMatrix &w);
// X: ldx % 4 == 0, 16-byte aligned.
hipError_t gemm_mfma(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias,
                     bool relu, const float *R, int ldr, hipStream_t st, float *ws = nullptr, size_t ws_bytes = 0);
constexpr size_t kGemmWorkspaceBytes = size_t(16) << 20;  // split-K partial sums
// Decoder-layer products of batches too large for the register GEMV: the split-K
// reduction folds in the residual add and the next LayerNorm (x += X W^T + bias;
// h = LayerNorm(x), N <= 4096), or the q / f16 K / V split of the fused QKV
// projection (q [M][d], caches at slot *step; qkv_tmp [M][3d] when K is not split).
hipError_t gemm_residual_ln(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, float *x,
                            const float *g, const float *b, float eps, float *h, hipStream_t st, float *ws,
                            size_t ws_bytes);
hipError_t gemm_qkv(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, int H, int hd, int slots,
                    const uint32_t *step, float *q, __half *kc, __half *vc, float *qkv_tmp, hipStream_t st, float *ws,
                    size_t ws_bytes);
hipError_t gemm_qkv(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, int H, int hd, int slots,
                    const uint32_t *step, float *q, float *kc, float *vc, float *qkv_tmp, hipStream_t st, float *ws,
                    size_t ws_bytes);
// ---- decode projections for batches of up to 64 rows, one launch each (k_dgemm.hip) ----
constexpr int kDgemmMaxRows = 64;
// Input LayerNorm from the statistics the residual stream's last writer left:
// stats [M][K / 16][2] (f64 sums of x and x^2 per 16 columns), gamma/beta [K].  With a
// DgemmLn, x is the residual stream in fragment order (frag_index, device.hpp).
struct DgemmLn {
    const double *stats;
    const float *g, *b;
    float eps;
};
bool dgemm_supported(const DevMatrix &w, int M);
// y[m][n] = (LN(x) or x)[m] . W[n] + bias[n], ReLU optional.  y_split: y is written as
// split fragments (frag_index, device.hpp), the A-operand form of the decode GEMMs; it
// then holds (M padded to 16) x N floats.
// resident: the LayerNorm projections of K = 1024 / 2048 may run the resident-X kernel
// (k_drx); false keeps k_dgemm's sums (the cross q whose fused launch k_dxattn must equal).
hipError_t dgemm_store(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias,
                       bool relu, float *y, int ldy, hipStream_t st, bool y_split = false, bool resident = true);
// xres[m][n] += x[m] . W[n] + bias[n] in place (xres: the residual stream, (M padded to
// 16) x N floats in fragment order), and stats_out [M][N / 16][2] of the new rows.
// x_split: x holds split fragments (else row-major f32 rows of ldx).
hipError_t dgemm_resid(const DevMatrix &w, const float *x, int ldx, int M, const float *bias, float *xres,
                       double *stats_out, hipStream_t st, bool x_split = false);
// The fused QKV projection: q [M][d] f32, K/V f16 into the caches [M][H][slots][hd] at *step.
hipError_t dgemm_qkv(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias, int H,
                     int hd, int slots, const uint32_t *step, float *q, __half *kc, __half *vc, hipStream_t st);
// The same with f32 caches (the generic decode path).
hipError_t dgemm_qkv(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias, int H,
                     int hd, int slots, const uint32_t *step, float *q, float *kc, float *vc, hipStream_t st);
// The cross attention of a decode step in one launch: q = LN(x) W^T + bias (x the residual
// stream, fragment order) and its attention over K/V [M][H][L][hd] (f16, lens[m] keys
// each); att [M][H hd] as split fragments, the cross out-projection's A operand.
bool dgemm_cross_attn_supported(const DevMatrix &w, int M, int H, int hd);
hipError_t dgemm_cross_attn(const DevMatrix &w, const float *x, int M, const DgemmLn &ln, const float *bias,
                            const __half *K, const __half *V, int H, int hd, int L, const uint32_t *lens, float *att,
                            hipStream_t st);
// The same over f32 K/V (the generic decoder).
hipError_t dgemm_cross_attn(const DevMatrix &w, const float *x, int M, const DgemmLn &ln, const float *bias,
                            const float *K, const float *V, int H, int hd, int L, const uint32_t *lens, float *att,
                            hipStream_t st);

// M <= 32 rows with X resident in LDS (K <= 1024 at M > 16, K <= 2048 at M <= 16).
bool gemm_rx_supported(const DevMatrix &w, int M);
// Greedy LM head for 4 < M <= 64: per-workgroup argmax partials pv/pi [M][parts] of
// X W^T (mask_id skipped), without storing the logits (M <= 32: X resident in LDS;
// 33..64: the wide-tile GEMM with an argmax epilogue).
bool gemm_argmax_supported(const DevMatrix &w, int M);
int gemm_argmax_parts(const DevMatrix &w, int M);
hipError_t gemm_argmax(const DevMatrix &w, const float *X, int ldx, int M, int mask_id, float *pv, uint32_t *pi,
                       int *parts, hipStream_t st);

// Streaming read of p[0, bytes) (measurement: the read ceiling), mode 0 / 1 / 2 =
// ordinary / non-temporal / direct-to-LDS 16-byte loads.
hipError_t stream_read(const void *p, size_t bytes, int mode, int grid, uint32_t *out, hipStream_t st);
// Row LayerNorm (biased variance): out = (x - mean) * rsqrt(var + eps) * g + b.
hipError_t layernorm(const float *x, int rows, int d, const float *g, const float *b, float eps, float *out,
                     hipStream_t st);
// The same with x in fragment order (frag_index, device.hpp; d % 16 == 0), out row-major.
hipError_t layernorm_frag(const float *x, int rows, int d, const float *g, const float *b, float eps, float *out,
                          hipStream_t st);
// x = x + y ; h = LayerNorm(x).  (bias already added to y by the producer)
hipError_t residual_ln(float *x, const float *y, int rows, int d, const float *g, const float *b, float eps, float *h,
                       hipStream_t st);
// ---- vocabulary shortlists (src/model.rs:555-603, kernels/malaga.cu:107-118, 229-326) ----
constexpr uint32_t kNoRow = 0xffffffffu;
// Decoder input copied from the source sentence: row r uses emb[r][row[r]] (f32) when
// row[r] != kNoRow, else the embedding matrix.
struct SrcEmb {
    const float *emb = nullptr;     // [b][S][d]
    const uint32_t *row = nullptr;  // [b]
    int S = 0;
};
// Shortlist form of greedy_finalize: the candidates of a row are the shortlist rows
// (partials pv/pi, indices < V1) then the source tokens (spv/spi [b][S], indices V1 + j).
// The winner maps to vocab_map[i] or src_ids[r][i - V1]; sl_row / src_row receive where
// the next input embedding is (shortlist row, or source position, else kNoRow).
struct SlFinalize {
    const uint32_t *vocab_map = nullptr;  // [V1]; null: no shortlist
    int V1 = 0;
    const float *spv = nullptr;
    const uint32_t *spi = nullptr;
    const uint32_t *src_ids = nullptr;    // [b][S]
    int S = 0;
    uint32_t *sl_row = nullptr, *src_row = nullptr;
};
// Logits of the source tokens (row_dots): spv[r][j] = h[r] . emb[r][j], spi = V1 + j;
// -inf where src_ids[r][j] == mask_id (mask_id >= 0).
hipError_t source_logits(const float *h, const float *emb, const uint32_t *src_ids, int b, int S, int d, int mask_id,
                         int V1, float *spv, uint32_t *spi, hipStream_t st);
// Rows of E as f32: out[r] = dequant(E[ids[r]]) (source-token embeddings).
hipError_t embed_rows(const DevMatrix &E, const uint32_t *ids, int rows, float *out, hipStream_t st);

// Decoder input: x = dequant(E[ids[r]]) * scale + pos[*step + base]; h = LayerNorm(x).
// src: rows whose input is a source-token embedding.  x_frag: x in fragment order
// (frag_index, device.hpp), h row-major.
hipError_t embed_pos_ln(const DevMatrix &E, const uint32_t *ids, int rows, const float *pos, const uint32_t *step,
                        uint32_t base, float scale, const float *g, const float *b, float eps, float *x, float *h,
                        hipStream_t st, const SrcEmb &src = SrcEmb{}, bool x_frag = false);
// Encoder input rows: x[r] = dequant(E[ids[r]]) * scale + pos[pidx[r]].
hipError_t embed_pos_rows(const DevMatrix &E, const uint32_t *ids, const uint32_t *pidx, int rows, const float *pos,
                          float scale, float *x, hipStream_t st);
// Splits qkv [b][3d] (bias included): q -> [b][H][hd] f32, k/v -> f16 caches
// [b][H][m][hd] at slot *step.
hipError_t qkv_split(const float *qkv, int b, int H, int hd, int m, const uint32_t *step, float *q, __half *kc,
                     __half *vc, hipStream_t st);
// The same into f32 caches (the generic decode path's K/V, src/model.rs:195-227).
hipError_t qkv_split(const float *qkv, int b, int H, int hd, int m, const uint32_t *step, float *q, float *kc,
                     float *vc, hipStream_t st);
// Single-query attention per (row, head) over f16 K/V [b][H][L][hd]: n = lens[row]
// if lens, else *step + 1.  out [b][H*hd].  Head sizes: attn_head_size_supported.
bool attn_head_size_supported(int hd);
hipError_t attn_decode(const float *q, const __half *K, const __half *V, int b, int H, int hd, int L,
                       const uint32_t *lens, const uint32_t *step, float *out, hipStream_t st, const uint32_t *rows = nullptr,
                       bool out_split = false);
// The same over f32 K/V (the generic decode path: candle KvCache and cross K/V in f32).
hipError_t attn_decode(const float *q, const float *K, const float *V, int b, int H, int hd, int L,
                       const uint32_t *lens, const uint32_t *step, float *out, hipStream_t st, const uint32_t *rows = nullptr,
                       bool out_split = false);
// rows (optional, [b][L]): cache row holding slot j of row b (beam reordering without copies).
// out_split: out is written as split fragments (frag_index, device.hpp), the input form
// of the decode GEMMs; out then holds (b padded to 16) x H*hd floats.
// Encoder self-attention over the packed rows (no padding rows): qkv [Mp][3d], row p a
// position of sentence rsent[p], whose keys are rows soff[i] .. soff[i] + lens[i] - 1;
// max_len >= every lens[i].  out [Mp][d].
hipError_t attn_prefill(const float *qkv, int Mp, int H, int hd, const uint32_t *soff, const uint32_t *rsent,
                        const uint32_t *lens, int max_len, float *out, hipStream_t st);
// kv [Mp][L][2d] f32 (the stacked cross K/V projection of L layers over the packed rows) ->
// f32 [b][H][s][hd]: packed row p is position prow[p] % s of sentence prow[p] / s; layer
// l's K at K0 + 2 l kv_elems, its V at K + kv_elems (kv_elems = b*s*d)
hipError_t split_cross_kv(const float *kv, int Mp, const uint32_t *prow, int s, int H, int hd, int L, float *K0,
                          size_t kv_elems, hipStream_t st);
// rows [r0, r0 + n) of w as a matrix of their own (block-major planes; no lane-major copy)
DevMatrix rows_view(const DevMatrix &w, int r0, int n);
// For each of `pairs` arrays (every layer's cross K and V): dst0 + p * dst_pair
// [.][H][S][hd] row r (< n_dst) <- src0 + p * src_pair [.][H][s][hd] row map[r] (row r if
// map is null), S >= s.  map is a device array; hd, the pair strides are multiples of 8
// values and the bases 16-byte aligned.  The source is f32 (the encoder's output); an f16
// destination receives it rounded to nearest even.
hipError_t copy_cross(const float *src0, size_t src_pair, const uint32_t *map, int n_dst, int H, int s, int hd,
                      __half *dst0, size_t dst_pair, int S, int pairs, hipStream_t st);
hipError_t copy_cross(const float *src0, size_t src_pair, const uint32_t *map, int n_dst, int H, int s, int hd,
                      float *dst0, size_t dst_pair, int S, int pairs, hipStream_t st);
// Argmax over logits [b][V] (row stride ldl) into pv/pi [b][parts].
hipError_t argmax_partial(const float *logits, int b, int V, int ldl, int mask_id, float *pv, uint32_t *pi,
                          int parts, hipStream_t st);
// Second argmax pass + greedy bookkeeping (kernels/malaga.cu:290-326 semantics):
// tok = finished ? pad : argmax ; finished |= tok == eos ; ids = tok ;
// out[row][*step] = tok ; ++*step.  outv (optional, [b][m]): outv[row][*step] = the
// winning logit (before the finished / pad rule).  err (optional): set to 1 when a row
// not yet finished has no finite logit.
hipError_t greedy_finalize(const float *pv, const uint32_t *pi, int parts, int b, uint8_t *finished, uint32_t *ids,
                           uint32_t *out, int m, uint32_t *step, uint32_t eos, uint32_t pad, hipStream_t st,
                           const SlFinalize &sl = SlFinalize{}, float *outv = nullptr, uint32_t *err = nullptr);
// Beam: per row log-softmax of logits [rows][V] and its top-k (k <= 8, ties -> lowest
// index): vals/idx [rows][k].  mask_id (>= 0) is treated as -inf.
hipError_t logsoftmax_topk(const float *logits, int rows, int V, int k, int mask_id, float *work, float *vals,
                           uint32_t *idx, hipStream_t st);
size_t logsoftmax_topk_scratch(int rows, int k);
// logsoftmax_topk with its work area in the library's static device array (no
// allocation; rows <= kStaticTopkRows).  The current device must be the stream's.
// Calls that overlap on one device share the array and race.
constexpr int kStaticTopkRows = 256;
hipError_t logsoftmax_topk_static(const float *logits, int rows, int V, int k, int mask_id, float *vals, uint32_t *idx,
                                  hipStream_t st);
// ---- fused decoder-step kernels (batch <= 4), k_step.hip ----
// True when the fused GEMV kernels (residual + LayerNorm prologue over d-wide rows)
// handle matrix w at batch nb.
bool step_fusable(const DevMatrix &w, int nb, int d);
// Number of partial sums step_attn_head writes for out-projection w (0: unsupported).
int step_head_parts(const DevMatrix &w, int nb, int d, int H, int hd, int L);
// True when step_qkv has an embedding prologue for (projection type, embedding type).
bool step_embed_supported(uint32_t proj_type, uint32_t emb_type);
// qkv projection; prologue = embedding rows (emb != null: x = E[ids] * scale +
// pos[*step + base]) or residual (x = x_in + y_in); x_out <- x (workgroup 0);
// h = LayerNorm(x); epilogue: q (rows < d), f16 K / V at cache slot *step.
hipError_t step_qkv(const DevMatrix &w, const float *bias, int nb, int d, const DevMatrix *emb, const uint32_t *ids,
                    const float *pos, uint32_t pos_base, float emb_scale, const float *x_in, const float *y_in,
                    float *x_out, const float *gamma, const float *beta, float eps, const uint32_t *step, float *q,
                    __half *kc, __half *vc, int H, int hd, int m, hipStream_t st, const SrcEmb &src = SrcEmb{});
// Attention of q over K/V [nb][H][L][hd] (lens: cross lengths, or null for *step + 1
// keys), times the out-projection w, as step_head_parts(...) partial sums
// part[p][nb][d] (bias not added): sum over p = attention . W^T.
hipError_t step_attn_head(const DevMatrix &w, int nb, int d, const float *q, const __half *K, const __half *V, int H,
                          int hd, int L, const uint32_t *lens, const uint32_t *step, float *part, hipStream_t st,
                          const uint32_t *rows = nullptr);
// x = x_in + sum_{p < P} part[p] + pbias ; x_out <- x ; y = LayerNorm(x) W^T + bias (relu).
hipError_t step_resid_proj(const DevMatrix &w, const float *bias, bool relu, int nb, int d, const float *x_in,
                           const float *part, int P, const float *pbias, float *x_out, const float *gamma,
                           const float *beta, float eps, float *y, hipStream_t st);
// step_resid_proj(cross_q) followed by step_attn_head(cross_out) in one launch:
// x = x_in + sum_{p < P} part_in[p] + pbias ; x_out <- x ; q = LayerNorm(x) Wq^T + bq ;
// part_out = the cross attention of q over K/V [nb][H][L][hd] (lens keys) times wo^T,
// step_head_parts(wo, ...) partial sums.  part_out must not alias part_in; P <= 8.
bool step_cross_fusable(const DevMatrix &wq, const DevMatrix &wo, int nb, int d, int H, int hd, int L, int P);
hipError_t step_cross_attn(const DevMatrix &wq, const float *bq, const DevMatrix &wo, int nb, int d, const float *x_in,
                           const float *part_in, int P, const float *pbias, float *x_out, const float *gamma,
                           const float *beta, float eps, const __half *K, const __half *V, int H, int hd, int L,
                           const uint32_t *lens, float *part_out, hipStream_t st);
// y = x W^T + bias, x [nb][K] in global memory.
hipError_t step_proj(const DevMatrix &w, const float *bias, int nb, const float *x, float *y, hipStream_t st);

// *p += 1 on the device.
hipError_t inc_u32(uint32_t *p, hipStream_t st);
// Fill n uint32 values (graph-safe replacement for hipMemsetAsync).
hipError_t fill_u32(uint32_t *p, uint32_t v, size_t n, hipStream_t st);

}  // namespace mlg
