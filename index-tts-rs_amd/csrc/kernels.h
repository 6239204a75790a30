// Host-side launchers of the gfx950 kernels.  Every launcher enqueues on `stream` and
// returns the launch status; shapes are validated by the caller (runtime.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace itts {

// kProEmbedLN: the input row is the step embedding mel_emb[ctl->tok] + mel_pos[ctl->pos]
// (block 0 stores it to x_out as the residual stream), then LayerNorm.
// kProAttn: the input row is the attention output, combined from the split partials of
// the decode attention (attn.part / attn.n_head / attn.max_splits, L from ctl).
enum Prologue : int { kProNone = 0, kProLN = 1, kProLNLN = 2, kProEmbedLN = 3, kProAttn = 4 };

struct AttnPartials {
  const float *part;  // [n_head][max_splits][66]: max, denominator, 64 outputs
  int n_head;
  int max_splits;
  int static_len;     // key count when ctl == nullptr
};
enum Epilogue : int { kEpiStore = 0, kEpiResid = 1, kEpiGelu = 2, kEpiQKV = 3 };

// Activations as the prefill GEMM reads them: x = hi + lo (fp16 planes, ~22 significant
// bits) and the row sums of each 64-column group (the MLX bias term needs sum_k x).
struct SplitAct {
  const uint16_t *hi, *lo;  // [M][K]
  const float *gs;          // [M][K/64]
};
struct SplitOut {
  uint16_t *hi, *lo;
  float *gs;
  SplitAct act() const { return SplitAct{hi, lo, gs}; }
};

// One sequence of a batched decode step: its control block, its cache bases (layer 0 of
// [layer][n_head][max_seq][64]) and its code output.
struct BatchSeq {
  DecodeCtl *ctl;
  void *k, *v;
  int32_t *codes;
};

// Where the QKV epilogue scatters: q -> q_out[M][d]; k, v -> this layer's cache
// [n_head][max_seq][64] at rows pos0.. .  With seqs set (batched decode), row m belongs
// to sequence m: its K/V row goes to seqs[m]'s cache at offset layer_off (elements) and
// position ctl->valid_len, and nothing is written for a finished sequence.
struct QkvDst {
  float *q_out;
  void *k_cache;
  void *v_cache;
  int max_seq;
  int pos0;
  int d_model;
  const BatchSeq *seqs;
  size_t layer_off;
};

struct GemvArgs {
  DevQL ql;
  const float *x;          // input row [K]
  const float *ln_w, *ln_b;    // LN (prologue kProLN / first LN of kProLNLN)
  const float *ln2_w, *ln2_b;  // second LN of kProLNLN
  float *y;                // output row [N] (store / gelu) or residual stream (resid)
  QkvDst qkv;
  const DecodeCtl *ctl;    // optional: early exit when done, cache row = valid_len
  const float *emb_tok, *emb_pos;  // kProEmbedLN tables (mel_emb, mel_pos)
  float *x_out;            // kProEmbedLN: residual stream written by block 0
  DecodeCtl *finish;       // optional: block 0 advances finish->valid_len after its rows
  AttnPartials attn;       // kProAttn
};

hipError_t launch_gemv(const GemvArgs &a, int bits, int ptype, int pro, int epi, int kvt,
                       hipStream_t s);

// Decode attention: q [n_head*64] against cache rows 0..L-1 with L = ctl->valid_len + 1
// (or static_len), 256 keys per split.  Each split writes its partial (max, denominator,
// 64 unnormalised outputs) to part [n_head][max_splits][66]; the consumer (the c_proj
// GEMV's kProAttn prologue) combines them.
int attn_decode_max_splits(int max_seq);
// Batched decode attention, one 16-wave block per (head, sequence), into the sequences'
// attention rows [B][d] in split form; finished sequences are skipped.
hipError_t launch_decode_batch_rows(const float *q, const BatchSeq *seqs, int B, size_t layer_off, int n_head,
                                    int max_seq, const SplitOut &out, int kvt, hipStream_t s);
// x[b] = mel_emb[tok_b] + mel_pos[pos_b] from the sequences' control blocks.
hipError_t launch_embed_batch(const BatchSeq *seqs, int B, const float *mel_emb, const float *mel_pos, int d, float *x,
                              hipStream_t s);
// valid_len += 1 for every sequence that is not finished.
hipError_t launch_advance_batch(const BatchSeq *seqs, int B, hipStream_t s);
hipError_t launch_attn_decode(const float *q, const void *kc, const void *vc, int n_head,
                              int max_seq, const DecodeCtl *ctl, int static_len, float *part,
                              int kvt, hipStream_t s);


// Row descriptors for the prefill embedding.
struct EmbedRow {
  int kind;  // 0 cond row, 1 text row, 2 Mel row
  int id;    // cond row index / token id
  int pos;   // positional index
};
hipError_t launch_embed_rows(const EmbedRow *rows, int T, const float *conds,
                             const float *text_emb, const float *lang_row,
                             const float *text_pos, const float *mel_emb,
                             const float *mel_pos, int d, float *x, hipStream_t s);

// LN of T rows [T][d] -> [T][d] in the GEMM's split form; with w2/b2 a second LN follows.
hipError_t launch_ln_rows(const float *x, const float *w, const float *b, int T, int d,
                          const SplitOut &y, hipStream_t s, const float *w2 = nullptr,
                          const float *b2 = nullptr);

// Attention probe: softmax probabilities of head `head` (none when < 0) for the query rows
// q0.. over the key columns [k0, k1): out [(rows - q0)][k1 - k0].
struct AttnProbe {
  int head, q0, k0, k1;
  float *out;
};
// Probe of M concatenated rows (row t attends to keys kstart[t]..t of the K/V
// [n_head][M][64]): writes only the probabilities, for rows p.q0..M-1.
hipError_t launch_attn_probe(const float *q, int M, const int *kstart, const void *kc, const void *vc, int n_head,
                             const AttnProbe &p, int kvt, hipStream_t s);
// Causal attention of T rows at cache positions base..base+T-1, one 64-lane block per
// (head, row) (short prompts); the output rows are written in the GEMM's split form.
hipError_t launch_attn_prefill(const float *q, int T, int base, const void *kc, const void *vc,
                               int n_head, int max_seq, const SplitOut &out, int kvt, hipStream_t s);
// Causal attention of T rows on the MFMA units: row t sits at position base + t of the
// K/V [n_head][ld][64] (bf16 or fp32) and attends to keys ks(t)..base + t, ks(t) =
// kstart[t] or 0; output rows in the GEMM's split form.
// With kv_split (attn_kv_split_halves(n_head, base + T) 16-bit values), K and V are split into
// fp16 hi/lo planes once per call instead of once per query tile.  With tile_order (a
// permutation of the ceil(T / 64) query tiles), grid row y runs query tile tile_order[y]:
// callers list the tiles with the most keys first so the short ones fill in behind them.
size_t attn_kv_split_halves(int n_head, int keys);
hipError_t launch_attn_flash(const float *q, int T, int base, const int *kstart, const void *kc, const void *vc,
                             int ld, int n_head, const SplitOut &out, int kvt, hipStream_t s,
                             uint16_t *kv_split = nullptr, const int *tile_order = nullptr);
// out[r] = log_softmax(logits[r])[codes[r]] for R rows of V logits.
hipError_t launch_log_softmax_pick(const float *logits, int R, int V, const int *codes, float *out, hipStream_t s);

// Prefill GEMM: y = x[M][K] . Wdeq^T + bias with the same epilogues as the GEMV.
// A LayerNorm folded into the product that follows it (few-row products, K <= 2048,
// K % 256 == 0): the product runs on gamma * x straight from the fp32 rows x [M][K] and its
// epilogue applies each row's statistics, rstd (sum - mean G[n]) + c[n], with G = W gamma
// and c = W beta + bias (launch_ln_fold), in place of sum + bias.
struct FoldIn {
  const float *x, *gamma, *G, *c;
};

// The same fold in the tiled product (any M): the input planes already hold gamma * x
// (written by the residual product before it, TileFoldOut), st[m][K/64] holds the mean
// and the sum of squared deviations of each 64-column group of row m of x, and the
// epilogue applies rstd (sum - mean G[n]) + c[n] with the row's statistics combined from
// its groups (equal-size groups: mean of the means, M2 = sum M2_g + 64 sum (mean_g - mean)^2).
struct TileFoldIn {
  const float2 *st;
  const float *G, *c;
};
// Residual epilogue that also writes the next folded LayerNorm's input from the updated
// rows x: gamma * x in split form (planes and group sums) and the group statistics of x.
struct TileFoldOut {
  SplitOut o;
  const float *gamma;
  float2 *st;       // [M][N/64]
};

struct GemmArgs {
  DevQL ql;
  SplitAct x;       // [M][K] (unused with fold.x)
  FoldIn fold;      // fold.x set: the input is LayerNorm(x) by the fold above
  TileFoldIn tfi;   // tfi.st set (tiled product, QKV or GELU epilogue): folded LayerNorm input
  TileFoldOut tfo;  // tfo.st set (tiled product, residual epilogue): write the next fold's input
  int M;
  float *y;         // [M][N] (store) or residual stream [M][N] (resid)
  SplitOut xo;      // gelu: the next GEMM's input [M][N] (N a multiple of 64)
  QkvDst qkv;
  // split-K partial tiles and per-tile arrival counters (zero between launches); split-K
  // is not used when they are absent or too small
  float *ws;
  size_t ws_floats;
  uint32_t *cnt;
  int cnt_words;
  int n_cu;         // compute units (grid sizing)
};
hipError_t launch_gemm(const GemmArgs &a, int bits, int ptype, int epi, int kvt, hipStream_t s);
// The tiled product uses 64 x 64 tiles up to this many rows, 128 x 128 tiles above.
constexpr int kGemmSmallTileRows = 512;
// Sets the LDS attributes of every GEMM instantiation (before any graph capture).
hipError_t gemm_init();
size_t gemm_ws_floats(int n_cu);
constexpr int kGemmCounters = 4096;

// fp32 rows [M][K] -> the GEMM's split form.
hipError_t launch_split_rows(const float *x, int M, int K, const SplitOut &o, hipStream_t s);

hipError_t launch_dequant(const DevQL &ql, int bits, int ptype, float *out, hipStream_t s);

// Persistent decode step (kernels_persist.hip): one launch of B blocks
// (one per CU) runs a whole decode step.  Exchange words are (epoch << 32 | fp32 bits).
constexpr int kCntStride = 32;  // one 128-byte line per head counter
struct PersistArgs {
  const DevLayer *layers;  // device array [n_layer]
  int n_layer, d, H, F, V, S, B;
  DevQL head;
  const float *ln_f_w, *ln_f_b, *fn_w, *fn_b;
  // LayerNorms folded into the QKV and c_fc products (ln_fold_layout): per layer
  // G = W.gamma and c = W.beta + bias of both products, fold_floats(d, F) floats a layer
  const float *fold;
  const float *mel_emb, *mel_pos;
  void *kc, *vc;           // cache bases [n_layer][H][max_seq][64], bf16 or f32 rows
  int max_seq;
  int kvt;                 // KvType of the rows
  DecodeCtl *ctl;
  // exchange arrays of 16-byte words (three values and an epoch), 16-byte aligned
  void *x_x, *x_qkv, *x_part, *x_attn, *x_mid, *x_f;
  uint32_t *cnt;           // [H * kCntStride] split counters (wrap at S; start at 0)
  uint32_t *err;           // nonzero after a timed-out wait
  float *logits;           // [V]
  uint32_t ep_stride;      // epochs per step: 8 * (n_layer + 1)
  // LDS region sizes (floats, multiples of 4): input row, normalised row (both long enough
  // for the dot products' padded layout: 4 floats after every 16-byte code chunk's
  // values), per-chunk partials, residual slice, row outputs, attention partials of one
  // head, one layer's staged parameters
  int xin_len, xn_len, part_len, own_len, out_len, pp_len, lp_len;
};
// A LayerNorm followed by a QuantizedLinear, y = W.((x - mu) * rstd * gamma + beta) + bias,
// equals rstd * (W.(gamma * x) - mu * G) + c with G = W.gamma and c = W.beta + bias, so
// the product can start on gamma * x before mu and rstd are known.  Per layer the fold
// buffer holds G and c of c_attn (ln_1) and of c_fc (ln_2):
//   [G_qkv 3d][c_qkv 3d][G_fc F][c_fc F]
__host__ __device__ inline size_t fold_floats(int d, int F) { return 6 * (size_t)d + 2 * (size_t)F; }
// G[o] = sum_k Wdeq[o][k] gamma[k] and c[o] = sum_k Wdeq[o][k] beta[k] + bias[o] for the N
// rows of ql (fp64 sums, rounded once), one wave per row.
hipError_t launch_ln_fold(const DevQL &ql, int bits, int ptype, const float *gamma, const float *beta, float *G,
                          float *c, hipStream_t s);
// Whether the persistent step supports this shape on B blocks; *S = attention splits.
// f32 rows also need persist_f32_v_floats() floats from the start of the block's LDS
// (input row, normalised row and partials: the host pads the partials to fit).
bool persist_supported(int d, int F, int V, int H, int n_layer, int max_seq, int B, int bits, int *S);
constexpr size_t kPersistMaxLds = 150 * 1024;
// LDS floats that f32 V rows of one attention split take: 512 per chunk of 8 keys.
inline int persist_f32_v_floats(int max_seq, int S) { return 512 * (((max_seq + S - 1) / S + 7) / 8); }
size_t persist_lds_bytes(const PersistArgs &a);
// 16-byte words of the exchange arrays x_x, x_qkv, x_part, x_attn, x_mid, x_f: total, and
// each array's offset in off[6].
size_t persist_exchange_words(int d, int F, int H, int S, int B, size_t off[6]);
// Whether one block of the persistent kernel with `lds` bytes of dynamic LDS fits a
// compute unit (threads, static + dynamic LDS).
hipError_t persist_fits(int bits, int ptype, int kvt, size_t lds, bool *fits);
hipError_t launch_decode_persist(PersistArgs a, int bits, int ptype, hipStream_t s);
// Raises the kernel's dynamic-LDS limit; once per process, outside stream capture.
hipError_t persist_init();

// Raises the sampler's dynamic-LDS limit; call once per process before any launch
// (never during stream capture).
hipError_t sampler_init();

// Device sampler (one block).  mode 0: API call on `logits` (penalised in place,
// token to *tok_out, rng advanced); mode 1: generate step driven by ctl.
hipError_t launch_sampler(float *logits, int n, const uint64_t *seen, DevSampling p,
                          uint64_t *rng, int32_t *tok_out, DecodeCtl *ctl, int32_t *codes,
                          int stop_tok, int mode, hipStream_t s);
// One sampler block per sequence of a batch: block b samples logits[b][n] with ps[b] into
// seqs[b]'s control block and codes (the generate loop's mode).  lds_top_k is the largest
// top_k of the batch (sets the LDS of the candidate sort).
hipError_t launch_sampler_batch(float *logits, int n, const DevSampling *ps, const BatchSeq *seqs, int B,
                                int stop_tok, int lds_top_k, bool any_sampled, hipStream_t s);

// Device ordinals the library accepts.
constexpr int kMaxDevices = 64;
// Staging area of the sampler's no-allocation entry point: a static device array (one per
// device, held until the process ends) with room for kStageMaxLogits logits, the seen-set
// words, the RNG state and the token.
constexpr int kStageMaxLogits = 9216;
struct SamplerStage {
  float *logits;   // [kStageMaxLogits]
  uint64_t *seen;  // [129]
  uint64_t *rng;
  int32_t *tok;
};
// Looks up the staging array's address on device dev, which must be the current device;
// later calls for the same device do nothing.
hipError_t sampler_stage_init(int dev);
// The staging area of device dev; false if sampler_stage_init has not run for it.
bool sampler_stage(int dev, SamplerStage *out);

// ---- Stage-2 CFM DiT estimator (kernels_cfm.hip); activations [B][T][C] fp32 ----
hipError_t cfm_temb(const float *t, int B, float *emb /*[B][256]*/, hipStream_t s);
hipError_t cfm_silu(const float *x, float *y, int n, hipStream_t s);
hipError_t cfm_bias_rows(float *C, int ldc, const float *bias, int rows, int cols, hipStream_t s);
hipError_t cfm_add_bias(float *C, int ldc, const float *bias, int rows, int cols, hipStream_t s);
hipError_t cfm_adaln(const float *x, float *y, int R, int T, int d, const float *mod, int ld_mod, const float *norm_w,
                     hipStream_t s);
hipError_t cfm_final_norm(const float *x, float *y, int R, int T, int d, const float *mod, hipStream_t s);
// rope (cos, sin) table [T][32][2] for positions 0..T-1
hipError_t cfm_rope_table(int T, float *tab, hipStream_t s);
// Key splits the attention uses for this shape on n_cu compute units (1..8); with more than
// one, part_o holds [S][B][T][d] and part_ml [S][B][H][T][2] floats.
int cfm_attn_splits(int B, int T, int H, int n_cu);
// kv_split: workspace of cfm_kv_split_halves(B, T, H) 16-bit values (K with rope and V as
// fp16 hi/lo planes, built once per call and shared by every query tile).
int cfm_kv_split_halves(int B, int T, int H);
// The MFMA GEMM's operand rules: K, lda, ldw multiples of 4 and A, W 16-byte aligned (the
// split and the launches reject anything else).
bool cfm_gemm_fits(const float *A, int lda, const float *W, int ldw, int K);
// The constant operand W [N][ldw] split once into fp16 hi/lo quads (cfm_split_weights_quads(N,
// K) uint4 at out, rows padded to 64 and k to 128 with zeros), and the products over them:
// cfm_gemm_split_w y[z] = A[z] W^T (+ bias) + beta y[z] for z < batch (row-major; A rows lda
// apart and allowed to overlap, batch strides sa / sy in floats) on the MFMA units with fp16
// hi/lo operands and fp32 accumulation (K, lda multiples of 4, A 16-byte aligned).
size_t cfm_split_weights_quads(int N, int K);
hipError_t cfm_split_weights(const float *W, int ldw, int N, int K, uint4 *out, hipStream_t s, int ilv = 0);
// act [M][ldo] = silu(A W1^T) * (A W3^T) for the packed W = [w1; w3] (2F rows) split with
// ilv = F: the SwiGLU in the product's epilogue (F a multiple of 32).
hipError_t cfm_gemm_swiglu(int M, int F, int K, const float *A, int lda, const uint4 *Wp, float *act, int ldo,
                           hipStream_t s);
hipError_t cfm_gemm_split_w(int batch, int M, int N, int K, const float *A, int lda, long sa, const uint4 *Wp,
                            float *y, int ldy, long sy, float beta, hipStream_t s, const float *bias = nullptr,
                            const float *yr = nullptr);
// The same product in fp32 FMAs for few rows (any M, any alignment; float4 loads when K,
// lda, ldw, sa, sw are multiples of 4 and A, W are 16-byte aligned); beta 0 never reads y.
// With bias (here and in cfm_gemm_split_w): y = A W^T + bias[n] + beta y; with yr, beta's
// old values come from yr (same layout as y) and y is written out of place.
hipError_t cfm_rows_gemm(int batch, int M, int N, int K, const float *A, int lda, long sa, const float *W, int ldw,
                         long sw, float *y, int ldy, long sy, float beta, hipStream_t s, const float *bias = nullptr,
                         const float *yr = nullptr);
hipError_t cfm_attention(const float *qkv, const float *rope_tab, int B, int T, int d, int H, float *out,
                         float *part_o, float *part_ml, uint16_t *kv_split, int n_cu, hipStream_t s);
hipError_t cfm_swiglu(const float *gu, int R, int F, float *out, hipStream_t s);
hipError_t cfm_gate(const float *acts, const float *in_b, const float *g, int ld_g, int R, int T, int d, float *act,
                    hipStream_t s);
hipError_t cfm_res_skip(const float *rs, const float *rs_b, int last, int R, int T, int d, int pad, float *h,
                        float *out, hipStream_t s);
hipError_t cfm_euler_prep(float *x, int C, int T, int T_ref, float *xt, float *merged, int MD, hipStream_t s);
hipError_t cfm_euler_update(float *x, const float *v, int C, int T, float dt, float cfg, hipStream_t s);
hipError_t cfm_static_tail(float *merged, int MD, int C, int d, int S, int T, const float *ref_mel, int T_ref,
                           const float *style, hipStream_t s);
hipError_t cfm_transpose_tc(const float *v, int B, int T, int C, float *out, hipStream_t s);
hipError_t cfm_pad_rows(const float *x, int B, int T, int d, int pad, float *hp, hipStream_t s);
hipError_t cfm_fill(float *p, int n, float v, hipStream_t s);

}  // namespace itts
