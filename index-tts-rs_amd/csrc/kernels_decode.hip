// Decode-path kernels for gfx950: batch-1 dequantising GEMV with fused LayerNorm
// prologue and bias / residual / GELU / QKV-scatter epilogues, split-K decode
// attention over the bf16 (or fp32) KV cache, and the step embedding.
//
// GEMV layout.  A wave owns R output rows.  Row o's codes are read as 16-byte chunks
// (16 int8 codes or 32 int4 codes) with consecutive lanes on consecutive chunks, so a
// wave issues fully coalesced 1 KiB loads.  The group affine is folded algebraically:
//   sum_k x_k (s q_k + b) = s * sum_k x_k q_k + b * sum_k x_k,
// with the per-chunk sums of x computed once per block in LDS.  All arithmetic is fp32.
#include "kernels.h"

namespace itts {

namespace {

constexpr int kGemvThreads = 256;
constexpr int kNcMax = 8;  // chunks per lane per row (K <= 8192 int8 / 16384 int4)

template <int BITS>
__device__ inline float chunk_dot(const uint4 c, const float *xc) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float acc = 0.0f;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 xv = *reinterpret_cast<const float4 *>(xc + 4 * i);
      acc += xv.x * (float)(w[i] & 0xffu);
      acc += xv.y * (float)((w[i] >> 8) & 0xffu);
      acc += xv.z * (float)((w[i] >> 16) & 0xffu);
      acc += xv.w * (float)(w[i] >> 24);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 xa = *reinterpret_cast<const float4 *>(xc + 8 * i);
      const float4 xb = *reinterpret_cast<const float4 *>(xc + 8 * i + 4);
      acc += xa.x * (float)(w[i] & 0xfu);
      acc += xa.y * (float)((w[i] >> 4) & 0xfu);
      acc += xa.z * (float)((w[i] >> 8) & 0xfu);
      acc += xa.w * (float)((w[i] >> 12) & 0xfu);
      acc += xb.x * (float)((w[i] >> 16) & 0xfu);
      acc += xb.y * (float)((w[i] >> 20) & 0xfu);
      acc += xb.z * (float)((w[i] >> 24) & 0xfu);
      acc += xb.w * (float)(w[i] >> 28);
    }
  }
  return acc;
}

template <int KVT>
__device__ inline void store_kv(void *cache, size_t idx, float v) {
  if constexpr (KVT == kKvBf16) {
    static_cast<uint16_t *>(cache)[idx] = (uint16_t)float_to_bf16_bits(v);
  } else {
    static_cast<float *>(cache)[idx] = v;
  }
}

template <int BITS, int PT, int PRO, int EPI, int KVT, int R>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  if (a.ctl != nullptr && a.ctl->done) return;
  extern __shared__ float smem[];
  constexpr int EPC = BITS == 8 ? 16 : 32;  // elements per 16-byte chunk
  const int K = a.ql.K, N = a.ql.N;
  const int nchunk = K / EPC;
  float *xl = smem;
  float *xsum = smem + K;
  float *red = xsum + nchunk;

  if constexpr (PRO == kProNone) {
    for (int i = threadIdx.x; i < K; i += kGemvThreads) xl[i] = a.x[i];
    __syncthreads();
  } else {
    layernorm_to_lds<kGemvThreads>(a.x, a.ln_w, a.ln_b, K, xl, red);
    if constexpr (PRO == kProLNLN) layernorm_lds_inplace<kGemvThreads>(xl, a.ln2_w, a.ln2_b, K, red);
  }
  for (int c = threadIdx.x; c < nchunk; c += kGemvThreads) {
    float s = 0.0f;
#pragma unroll 8
    for (int i = 0; i < EPC; i++) s += xl[c * EPC + i];
    xsum[c] = s;
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * (kGemvThreads / 64) + wave) * R;
  const size_t row_bytes = (size_t)K * BITS / 8;
  const int G = K / kGroup;

  uint4 cw[R][kNcMax];
  float2 pr[R][kNcMax];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = row0 + r;
#pragma unroll
    for (int j = 0; j < kNcMax; j++) {
      const int c = lane + 64 * j;
      if (row < N && c < nchunk) {
        cw[r][j] = *reinterpret_cast<const uint4 *>(a.ql.codes + row * row_bytes + (size_t)c * 16);
        pr[r][j] = load_param<PT>(a.ql.params, (size_t)row * G + (size_t)c * EPC / kGroup);
      } else {
        cw[r][j] = make_uint4(0, 0, 0, 0);
        pr[r][j] = make_float2(0.0f, 0.0f);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = row0 + r;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kNcMax; j++) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        const float d = chunk_dot<BITS>(cw[r][j], xl + c * EPC);
        acc += pr[r][j].x * d + pr[r][j].y * xsum[c];
      }
    }
    acc = wave_sum(acc);
    if (lane == 0 && row < N) {
      const float v = acc + a.ql.bias[row];
      if constexpr (EPI == kEpiStore) {
        a.y[row] = v;
      } else if constexpr (EPI == kEpiResid) {
        a.y[row] = a.y[row] + v;
      } else if constexpr (EPI == kEpiGelu) {
        a.y[row] = gelu_tanh(v);
      } else {
        const int d = a.qkv.d_model;
        const int pos = a.ctl != nullptr ? a.ctl->valid_len : a.qkv.pos0;
        if (row < d) {
          a.qkv.q_out[row] = v;
        } else {
          const int idx = row < 2 * d ? row - d : row - 2 * d;
          const int h = idx >> 6, e = idx & 63;
          const size_t ci = ((size_t)h * a.qkv.max_seq + pos) * kHeadDim + e;
          store_kv<KVT>(row < 2 * d ? a.qkv.k_cache : a.qkv.v_cache, ci, v);
        }
      }
    }
  }
}

template <int BITS, int PT, int PRO, int EPI, int KVT>
hipError_t gemv_dispatch_r(const GemvArgs &a, hipStream_t s) {
  const int K = a.ql.K, N = a.ql.N;
  const int EPC = BITS == 8 ? 16 : 32;
  const size_t lds = sizeof(float) * ((size_t)K + K / EPC + 8);
  const int waves = kGemvThreads / 64;
  // Rows per wave: 4 when that still gives >= 256 blocks, else 1.
  if ((N + waves * 4 - 1) / (waves * 4) >= 256) {
    const int blocks = (N + waves * 4 - 1) / (waves * 4);
    hipLaunchKernelGGL((gemv_kernel<BITS, PT, PRO, EPI, KVT, 4>), dim3(blocks), dim3(kGemvThreads),
                       lds, s, a);
  } else {
    const int blocks = (N + waves - 1) / waves;
    hipLaunchKernelGGL((gemv_kernel<BITS, PT, PRO, EPI, KVT, 1>), dim3(blocks), dim3(kGemvThreads),
                       lds, s, a);
  }
  return hipGetLastError();
}

template <int BITS, int PT>
hipError_t gemv_dispatch_pe(const GemvArgs &a, int pro, int epi, int kvt, hipStream_t s) {
  if (pro == kProLN && epi == kEpiQKV) {
    return kvt == kKvBf16 ? gemv_dispatch_r<BITS, PT, kProLN, kEpiQKV, kKvBf16>(a, s)
                          : gemv_dispatch_r<BITS, PT, kProLN, kEpiQKV, kKvF32>(a, s);
  }
  if (pro == kProNone && epi == kEpiResid) return gemv_dispatch_r<BITS, PT, kProNone, kEpiResid, 0>(a, s);
  if (pro == kProLN && epi == kEpiGelu) return gemv_dispatch_r<BITS, PT, kProLN, kEpiGelu, 0>(a, s);
  if (pro == kProLNLN && epi == kEpiStore) return gemv_dispatch_r<BITS, PT, kProLNLN, kEpiStore, 0>(a, s);
  if (pro == kProNone && epi == kEpiStore) return gemv_dispatch_r<BITS, PT, kProNone, kEpiStore, 0>(a, s);
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------
// Attention
// ---------------------------------------------------------------------------------

template <int KVT>
__device__ inline void load_row64(const void *base, size_t row, float *out) {
  if constexpr (KVT == kKvBf16) {
    const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + row * 64);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint4 u = p[i];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
        out[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    }
  } else {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(base) + row * 64);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 f = p[i];
      out[4 * i] = f.x;
      out[4 * i + 1] = f.y;
      out[4 * i + 2] = f.z;
      out[4 * i + 3] = f.w;
    }
  }
}

template <int KVT>
__device__ inline float load_elem(const void *base, size_t idx) {
  if constexpr (KVT == kKvBf16) {
    return __uint_as_float((uint32_t) static_cast<const uint16_t *>(base)[idx] << 16);
  } else {
    return static_cast<const float *>(base)[idx];
  }
}

// One wave: online-softmax attention of query q (64 values, global) over keys j0..j1-1
// of one head's cache slice (rows of 64).  Returns the running max m, the denominator
// l and, in lane e, the unnormalised output o[e].
template <int KVT>
__device__ inline void attn_range(const float *q, const void *kh, const void *vh, int j0, int j1,
                                  float &m, float &l, float &o, float *p_lds) {
  const int lane = threadIdx.x & 63;
  float qr[64];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float4 v = reinterpret_cast<const float4 *>(q)[i];
    qr[4 * i] = v.x;
    qr[4 * i + 1] = v.y;
    qr[4 * i + 2] = v.z;
    qr[4 * i + 3] = v.w;
  }
  m = -INFINITY;
  l = 0.0f;
  o = 0.0f;
  for (int t0 = j0; t0 < j1; t0 += 64) {
    const int j = t0 + lane;
    float sc = -INFINITY;
    if (j < j1) {
      float kr[64];
      load_row64<KVT>(kh, (size_t)j, kr);
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < 64; e++) dot += qr[e] * kr[e];
      sc = dot * 0.125f;
    }
    const float mt = wave_max(sc);
    const float mn = fmaxf(m, mt);
    const float p = (j < j1) ? __expf(sc - mn) : 0.0f;
    const float corr = (m == -INFINITY) ? 0.0f : __expf(m - mn);
    l = l * corr + wave_sum(p);
    p_lds[lane] = p;
    __syncthreads();
    o *= corr;
    const int cnt = min(64, j1 - t0);
    for (int jj = 0; jj < cnt; jj++) o += p_lds[jj] * load_elem<KVT>(vh, (size_t)(t0 + jj) * 64 + lane);
    __syncthreads();
    m = mn;
  }
}

template <int KVT>
__global__ __launch_bounds__(64) void attn_decode_split_kernel(const float *q, const void *kc,
                                                               const void *vc, int max_seq,
                                                               const DecodeCtl *ctl, int static_len,
                                                               int chunk, float *part) {
  if (ctl != nullptr && ctl->done) return;
  __shared__ float p_lds[64];
  const int h = blockIdx.x, s = blockIdx.y, S = gridDim.y;
  const int L = ctl != nullptr ? ctl->valid_len + 1 : static_len;
  const int j0 = s * chunk, j1 = min(L, j0 + chunk);
  float *out = part + ((size_t)h * S + s) * 66;
  const int lane = threadIdx.x;
  if (j0 >= L) {
    if (lane == 0) {
      out[0] = -INFINITY;
      out[1] = 0.0f;
    }
    out[2 + lane] = 0.0f;
    return;
  }
  const size_t hb = (size_t)h * max_seq * 64;
  const void *kh = KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(kc) + hb)
                                  : (const void *)(static_cast<const float *>(kc) + hb);
  const void *vh = KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(vc) + hb)
                                  : (const void *)(static_cast<const float *>(vc) + hb);
  float m, l, o;
  attn_range<KVT>(q + h * 64, kh, vh, j0, j1, m, l, o, p_lds);
  if (lane == 0) {
    out[0] = m;
    out[1] = l;
  }
  out[2 + lane] = o;
}

__global__ __launch_bounds__(64) void attn_combine_kernel(const float *part, int S,
                                                          const DecodeCtl *ctl, float *out) {
  if (ctl != nullptr && ctl->done) return;
  const int h = blockIdx.x, e = threadIdx.x;
  const float *p = part + (size_t)h * S * 66;
  float M = -INFINITY;
  for (int s = 0; s < S; s++) M = fmaxf(M, p[s * 66]);
  float den = 0.0f, num = 0.0f;
  for (int s = 0; s < S; s++) {
    const float ms = p[s * 66];
    if (ms == -INFINITY) continue;
    const float w = __expf(ms - M);
    den += p[s * 66 + 1] * w;
    num += p[s * 66 + 2 + e] * w;
  }
  out[h * 64 + e] = num / den;
}

template <int KVT>
__global__ __launch_bounds__(64) void attn_prefill_kernel(const float *q, int base, const void *kc,
                                                          const void *vc, int max_seq, int d,
                                                          float *out) {
  __shared__ float p_lds[64];
  const int h = blockIdx.x, t = blockIdx.y;
  const size_t hb = (size_t)h * max_seq * 64;
  const void *kh = KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(kc) + hb)
                                  : (const void *)(static_cast<const float *>(kc) + hb);
  const void *vh = KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(vc) + hb)
                                  : (const void *)(static_cast<const float *>(vc) + hb);
  float m, l, o;
  attn_range<KVT>(q + (size_t)t * d + h * 64, kh, vh, 0, base + t + 1, m, l, o, p_lds);
  out[(size_t)t * d + h * 64 + threadIdx.x] = o / l;
}

// ---------------------------------------------------------------------------------
// Embeddings and LayerNorm rows
// ---------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void embed_step_kernel(const float *mel_emb, const float *mel_pos,
                                                         const DecodeCtl *ctl, int d, float *x) {
  if (ctl->done) return;
  const float *me = mel_emb + (size_t)ctl->tok * d;
  const float *mp = mel_pos + (size_t)ctl->pos * d;
  for (int i = threadIdx.x; i < d; i += 256) x[i] = me[i] + mp[i];
}

__global__ __launch_bounds__(256) void embed_rows_kernel(const EmbedRow *rows, const float *conds,
                                                         const float *text_emb, const float *lang_row,
                                                         const float *text_pos, const float *mel_emb,
                                                         const float *mel_pos, int d, float *x) {
  const EmbedRow r = rows[blockIdx.x];
  float *dst = x + (size_t)blockIdx.x * d;
  if (r.kind == 0) {
    const float *src = conds + (size_t)r.id * d;
    for (int i = threadIdx.x; i < d; i += 256) dst[i] = src[i];
  } else if (r.kind == 1) {
    const float *te = text_emb + (size_t)r.id * d;
    const float *tp = text_pos + (size_t)r.pos * d;
    for (int i = threadIdx.x; i < d; i += 256) dst[i] = (te[i] + lang_row[i]) + tp[i];
  } else {
    const float *me = mel_emb + (size_t)r.id * d;
    const float *mp = mel_pos + (size_t)r.pos * d;
    for (int i = threadIdx.x; i < d; i += 256) dst[i] = me[i] + mp[i];
  }
}

__global__ __launch_bounds__(256) void ln_rows_kernel(const float *x, const float *w, const float *b,
                                                      int d, float *y) {
  extern __shared__ float smem[];
  float *red = smem + d;
  layernorm_to_lds<256>(x + (size_t)blockIdx.x * d, w, b, d, smem, red);
  for (int i = threadIdx.x; i < d; i += 256) y[(size_t)blockIdx.x * d + i] = smem[i];
}

__global__ void step_finish_kernel(DecodeCtl *ctl) {
  if (!ctl->done) ctl->valid_len += 1;
}

}  // namespace

hipError_t launch_gemv(const GemvArgs &a, int bits, int ptype, int pro, int epi, int kvt,
                       hipStream_t s) {
  const int epc = bits == 8 ? 16 : 32;
  if (a.ql.K % kGroup != 0 || a.ql.K / epc > 64 * kNcMax) return hipErrorInvalidValue;
  if (bits == 8) {
    return ptype == kParamF16 ? gemv_dispatch_pe<8, kParamF16>(a, pro, epi, kvt, s)
                              : gemv_dispatch_pe<8, kParamF32>(a, pro, epi, kvt, s);
  }
  if (bits == 4) {
    return ptype == kParamF16 ? gemv_dispatch_pe<4, kParamF16>(a, pro, epi, kvt, s)
                              : gemv_dispatch_pe<4, kParamF32>(a, pro, epi, kvt, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_attn_decode(const float *q, const void *kc, const void *vc, int n_head,
                              int max_seq, const DecodeCtl *ctl, int static_len, float *part,
                              int max_splits, int chunk, float *out, int kvt, hipStream_t s) {
  dim3 grid(n_head, max_splits);
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL(attn_decode_split_kernel<kKvBf16>, grid, dim3(64), 0, s, q, kc, vc, max_seq,
                       ctl, static_len, chunk, part);
  } else {
    hipLaunchKernelGGL(attn_decode_split_kernel<kKvF32>, grid, dim3(64), 0, s, q, kc, vc, max_seq,
                       ctl, static_len, chunk, part);
  }
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_head), dim3(64), 0, s, part, max_splits, ctl, out);
  return hipGetLastError();
}

hipError_t launch_attn_prefill(const float *q, int T, int base, const void *kc, const void *vc,
                               int n_head, int max_seq, float *out, int kvt, hipStream_t s) {
  dim3 grid(n_head, T);
  const int d = n_head * 64;
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL(attn_prefill_kernel<kKvBf16>, grid, dim3(64), 0, s, q, base, kc, vc, max_seq, d,
                       out);
  } else {
    hipLaunchKernelGGL(attn_prefill_kernel<kKvF32>, grid, dim3(64), 0, s, q, base, kc, vc, max_seq, d,
                       out);
  }
  return hipGetLastError();
}

hipError_t launch_embed_step(const float *mel_emb, const float *mel_pos, const DecodeCtl *ctl,
                             int d, float *x, hipStream_t s) {
  hipLaunchKernelGGL(embed_step_kernel, dim3(1), dim3(256), 0, s, mel_emb, mel_pos, ctl, d, x);
  return hipGetLastError();
}

hipError_t launch_embed_rows(const EmbedRow *rows, int T, const float *conds,
                             const float *text_emb, const float *lang_row,
                             const float *text_pos, const float *mel_emb,
                             const float *mel_pos, int d, float *x, hipStream_t s) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3(T), dim3(256), 0, s, rows, conds, text_emb, lang_row,
                     text_pos, mel_emb, mel_pos, d, x);
  return hipGetLastError();
}

hipError_t launch_ln_rows(const float *x, const float *w, const float *b, int T, int d,
                          float *y, hipStream_t s) {
  hipLaunchKernelGGL(ln_rows_kernel, dim3(T), dim3(256), sizeof(float) * (d + 8), s, x, w, b, d, y);
  return hipGetLastError();
}

hipError_t launch_step_finish(DecodeCtl *ctl, hipStream_t s) {
  hipLaunchKernelGGL(step_finish_kernel, dim3(1), dim3(1), 0, s, ctl);
  return hipGetLastError();
}

}  // namespace itts
