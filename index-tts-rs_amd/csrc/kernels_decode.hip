// Decode-path kernels for gfx950: batch-1 dequantising GEMV with fused LayerNorm /
// embedding prologues and bias / residual / GELU / QKV-scatter epilogues, split-K decode
// attention with an in-kernel combine, and the prefill helpers (row embedding, row
// LayerNorm, causal attention).
//
// GEMV layout.  A wave owns R output rows.  Row o's codes are read as 16-byte chunks
// (16 int8 codes or 32 int4 codes), consecutive lanes on consecutive chunks, so a wave
// issues fully coalesced 1 KiB loads.  Every weight load of the block is issued before
// the prologue (LayerNorm of the input row, or the step embedding), so the prologue runs
// while the codes are in flight.  The group affine is folded algebraically:
//   sum_k x_k (s q_k + b) = s * sum_k x_k q_k + b * sum_k x_k,
// with the per-chunk sums of x formed once per block in LDS.  All arithmetic is fp32.
#include "kernels.h"

namespace itts {

namespace {

constexpr int kGemvThreads = 256;
constexpr int kAttnKeys = 256;  // keys per decode-attention split

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

// NC: 16-byte chunks per lane per row (ceil(K / elements-per-chunk / 64)).
template <int BITS, int PT, int PRO, int EPI, int KVT, int R, int NC>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  if (a.ctl != nullptr && a.ctl->done) return;
  extern __shared__ float smem[];
  constexpr int EPC = BITS == 8 ? 16 : 32;  // elements per 16-byte chunk
  constexpr int XPT = NC * EPC * 64 / kGemvThreads;  // input values per thread (upper bound)
  const int K = a.ql.K, N = a.ql.N;
  const int nchunk = K / EPC;
  const int tid = threadIdx.x;
  float *xl = smem;
  float *xsum = smem + K;
  float *red = xsum + nchunk;

  // 1. input row first: it is needed before the weights, and loads complete in issue order
  float xr[XPT];
  if constexpr (PRO == kProEmbedLN) {
    const float *me = a.emb_tok + (size_t)a.ctl->tok * K;
    const float *mp = a.emb_pos + (size_t)a.ctl->pos * K;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int idx = tid + kGemvThreads * i;
      xr[i] = idx < K ? me[idx] + mp[idx] : 0.0f;
    }
  } else if constexpr (PRO == kProAttn) {
    // combine the attention splits: out[h][e] = sum_s o_s[e] e^{m_s-M} / sum_s l_s e^{m_s-M}.
    // Stage A: per (head, split) the scaled weight e^{m_s-M}/den into LDS.
    const int L = a.ctl != nullptr ? a.ctl->valid_len + 1 : a.attn.static_len;
    const int S = (L + kAttnKeys - 1) / kAttnKeys;
    const int H = a.attn.n_head, MS = a.attn.max_splits;
    float *wts = red + 8;  // [H][S]
    for (int h = tid; h < H; h += kGemvThreads) {
      const float *ph = a.attn.part + (size_t)h * MS * 66;
      float M = -INFINITY;
      for (int s = 0; s < S; s++) M = fmaxf(M, ph[s * 66]);
      float den = 0.0f;
      for (int s = 0; s < S; s++) den += ph[s * 66 + 1] * __expf(ph[s * 66] - M);
      const float inv = 1.0f / den;
      for (int s = 0; s < S; s++) wts[h * S + s] = __expf(ph[s * 66] - M) * inv;
    }
    __syncthreads();
    // Stage B: the weighted sum of this thread's elements (loads issued before the weights)
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int idx = tid + kGemvThreads * i;
      float acc = 0.0f;
      if (idx < K) {
        const int h = idx >> 6, e = idx & 63;
        const float *ph = a.attn.part + (size_t)h * MS * 66 + 2 + e;
        for (int s = 0; s < S; s++) acc += ph[s * 66] * wts[h * S + s];
      }
      xr[i] = acc;
    }
  } else {
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int idx = tid + kGemvThreads * i;
      xr[i] = idx < K ? a.x[idx] : 0.0f;
    }
  }

  // 2. weight loads
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * (kGemvThreads / 64) + wave) * R;
  const size_t row_bytes = (size_t)K * BITS / 8;
  const int G = K / kGroup;
  uint4 cw[R][NC];
  float2 pr[R][NC];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = row0 + r;
#pragma unroll
    for (int j = 0; j < NC; j++) {
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

  // 3. prologue: the input row into LDS (waits for the input loads only), then LayerNorm
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int idx = tid + kGemvThreads * i;
    if (idx < K) xl[idx] = xr[i];
  }
  if constexpr (PRO == kProEmbedLN) {
    // x = mel_emb[tok] + mel_pos[pos] (gpt.rs:720-725); block 0 keeps it as the residual
    if (blockIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < XPT; i++) {
        const int idx = tid + kGemvThreads * i;
        if (idx < K) a.x_out[idx] = xr[i];
      }
    }
  }
  __syncthreads();
  if constexpr (PRO == kProLN || PRO == kProLNLN || PRO == kProEmbedLN) {
    layernorm_lds_inplace<kGemvThreads>(xl, a.ln_w, a.ln_b, K, red);
    if constexpr (PRO == kProLNLN) layernorm_lds_inplace<kGemvThreads>(xl, a.ln2_w, a.ln2_b, K, red);
  }
  for (int c = threadIdx.x; c < nchunk; c += kGemvThreads) {
    float s = 0.0f;
#pragma unroll 8
    for (int i = 0; i < EPC; i++) s += xl[c * EPC + i];
    xsum[c] = s;
  }
  __syncthreads();

  // 3. dot products, wave reduction, epilogue
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = row0 + r;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; j++) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        const float d = chunk_dot<BITS>(cw[r][j], xl + c * EPC);
        acc += pr[r][j].x * d + pr[r][j].y * xsum[c];
      }
    }
    acc = wave64_sum_dpp(acc);
    if (lane == 0 && row < N) {
      const float v = acc + a.ql.bias[row];
      if constexpr (EPI == kEpiStore) {
        a.y[row] = v;
      } else if constexpr (EPI == kEpiResid) {
        a.y[row] = a.y[row] + v;
      } else if constexpr (EPI == kEpiGelu) {
        a.y[row] = gelu_tanh_exp(v);
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
  // the head of a decode step closes the step: the cache now holds one more row
  if (a.finish != nullptr && blockIdx.x == 0 && threadIdx.x == 0) a.finish->valid_len += 1;
}

template <int BITS, int PT, int PRO, int EPI, int KVT, int NC>
hipError_t gemv_dispatch_r(const GemvArgs &a, hipStream_t s) {
  const int K = a.ql.K, N = a.ql.N;
  const int EPC = BITS == 8 ? 16 : 32;
  const size_t attn_wts = PRO == kProAttn ? (size_t)a.attn.n_head * a.attn.max_splits : 0;
  const size_t lds = sizeof(float) * ((size_t)K + K / EPC + 8 + attn_wts);
  const int waves = kGemvThreads / 64;
  // two rows per wave when that still leaves >= 2 blocks per CU, else one
  if ((N + waves * 2 - 1) / (waves * 2) >= 448) {
    const int blocks = (N + waves * 2 - 1) / (waves * 2);
    hipLaunchKernelGGL((gemv_kernel<BITS, PT, PRO, EPI, KVT, 2, NC>), dim3(blocks), dim3(kGemvThreads),
                       lds, s, a);
  } else {
    const int blocks = (N + waves - 1) / waves;
    hipLaunchKernelGGL((gemv_kernel<BITS, PT, PRO, EPI, KVT, 1, NC>), dim3(blocks), dim3(kGemvThreads),
                       lds, s, a);
  }
  return hipGetLastError();
}

template <int BITS, int PT, int PRO, int EPI, int KVT>
hipError_t gemv_dispatch_nc(const GemvArgs &a, hipStream_t s) {
  const int epc = BITS == 8 ? 16 : 32;
  const int nc = (a.ql.K / epc + 63) / 64;
  switch (nc) {
    case 1: return gemv_dispatch_r<BITS, PT, PRO, EPI, KVT, 1>(a, s);
    case 2: return gemv_dispatch_r<BITS, PT, PRO, EPI, KVT, 2>(a, s);
    case 3: return gemv_dispatch_r<BITS, PT, PRO, EPI, KVT, 3>(a, s);
    case 4:
    case 5: return gemv_dispatch_r<BITS, PT, PRO, EPI, KVT, 5>(a, s);
    case 6:
    case 7:
    case 8: return gemv_dispatch_r<BITS, PT, PRO, EPI, KVT, 8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <int BITS, int PT>
hipError_t gemv_dispatch_pe(const GemvArgs &a, int pro, int epi, int kvt, hipStream_t s) {
  if (epi == kEpiQKV && (pro == kProLN || pro == kProEmbedLN)) {
    if (pro == kProLN)
      return kvt == kKvBf16 ? gemv_dispatch_nc<BITS, PT, kProLN, kEpiQKV, kKvBf16>(a, s)
                            : gemv_dispatch_nc<BITS, PT, kProLN, kEpiQKV, kKvF32>(a, s);
    return kvt == kKvBf16 ? gemv_dispatch_nc<BITS, PT, kProEmbedLN, kEpiQKV, kKvBf16>(a, s)
                          : gemv_dispatch_nc<BITS, PT, kProEmbedLN, kEpiQKV, kKvF32>(a, s);
  }
  if (pro == kProNone && epi == kEpiResid) return gemv_dispatch_nc<BITS, PT, kProNone, kEpiResid, 0>(a, s);
  if (pro == kProAttn && epi == kEpiResid) return gemv_dispatch_nc<BITS, PT, kProAttn, kEpiResid, 0>(a, s);
  if (pro == kProLN && epi == kEpiGelu) return gemv_dispatch_nc<BITS, PT, kProLN, kEpiGelu, 0>(a, s);
  if (pro == kProLNLN && epi == kEpiStore) return gemv_dispatch_nc<BITS, PT, kProLNLN, kEpiStore, 0>(a, s);
  if (pro == kProNone && epi == kEpiStore) return gemv_dispatch_nc<BITS, PT, kProNone, kEpiStore, 0>(a, s);
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------
// Decode attention: grid (head, split), 256 keys per split (4 waves x 64 keys, each wave
// one tile of attn_range below).  Each block writes its partial (max, denominator, 64
// unnormalised outputs); the c_proj GEMV that consumes the attention output combines the
// partials in its prologue.
// ---------------------------------------------------------------------------------

template <int KVT>
__device__ inline const void *head_base(const void *c, size_t off) {
  return KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(c) + off)
                        : (const void *)(static_cast<const float *>(c) + off);
}

// Eight consecutive elements of a cache row, held in the cache dtype until used.
template <int KVT>
struct Row8 {
  uint32_t w[KVT == kKvBf16 ? 4 : 8];
  // through the global address space: a cache pointer read from a sequence descriptor is
  // generic to the compiler, and generic (flat) loads also count against the LDS counter
  typedef unsigned int gu32x4 __attribute__((ext_vector_type(4)));
  typedef const __attribute__((address_space(1))) gu32x4 *gptr;
  __device__ __forceinline__ void load(const void *base, size_t row, int c0) {
    if constexpr (KVT == kKvBf16) {
      const gu32x4 u = *(gptr)(static_cast<const uint16_t *>(base) + row * 64 + c0);
      w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w;
    } else {
      const gptr p = (gptr)(static_cast<const float *>(base) + row * 64 + c0);
      const gu32x4 u0 = p[0], u1 = p[1];
      w[0] = u0.x; w[1] = u0.y; w[2] = u0.z; w[3] = u0.w;
      w[4] = u1.x; w[5] = u1.y; w[6] = u1.z; w[7] = u1.w;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < (KVT == kKvBf16 ? 4 : 8); i++) w[i] = 0u;
  }
  __device__ __forceinline__ float at(int e) const {
    if constexpr (KVT == kKvBf16)
      return __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
    else
      return __uint_as_float(w[e]);
  }
};

// Score (q.k / 8) of key row `kr`, whose dims 8 dc .. 8 dc + 7 this lane holds against
// q's in qa, qb: the lane's partial dot, summed over the key's eight lanes (xor 1, xor 2,
// then the 8-lane mirror; both lanes of each pair form the same sum, so all eight lanes
// hold one bit-identical score).  Every lane of the wave must be active.
template <int KVT>
__device__ __forceinline__ float row_score(const float4 &qa, const float4 &qb, const Row8<KVT> &kr) {
  float t = qa.x * kr.at(0) + qa.y * kr.at(1) + qa.z * kr.at(2) + qa.w * kr.at(3) +
            (qb.x * kr.at(4) + qb.y * kr.at(5) + qb.z * kr.at(6) + qb.w * kr.at(7));
  t += dpp_pair<0xB1>(t);
  t += dpp_pair<0x4E>(t);
  t += dpp_pair<0x141>(t);
  return t * 0.125f;
}

// One wave's online-softmax state over one query row, 64 keys a tile.  Lane = (key group
// kg = lane / 8, dims 8 (lane % 8) .. +7): a lane holds keys kg, kg + 8, .. of the tile, K and
// V rows both spread over eight adjacent lanes (16 bytes each, so a load instruction reads
// eight whole rows); probabilities stay in the lane that holds the key, and the eight key
// groups are added once at the end (finish: dimension `lane` of the unnormalised output).
template <int KVT>
struct AttnRun {
  float4 qa, qb;
  float m, l, acc[8];
  __device__ __forceinline__ void init(const float *q) {
    const int dc = threadIdx.x & 7;
    qa = reinterpret_cast<const float4 *>(q)[2 * dc];
    qb = reinterpret_cast<const float4 *>(q)[2 * dc + 1];
    m = -INFINITY;
    l = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
  }
  // keys t0 .. min(t0 + 64, j1) - 1, rows kr/vr as this lane holds them (zero past j1)
  __device__ __forceinline__ void tile(int t0, int j1, const Row8<KVT> (&kr)[8], const Row8<KVT> (&vr)[8]) {
    const int kg = (threadIdx.x & 63) >> 3;
    float sc[8], mt = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const float v = row_score<KVT>(qa, qb, kr[jj]);
      sc[jj] = t0 + kg + 8 * jj < j1 ? v : -INFINITY;
      mt = fmaxf(mt, sc[jj]);
    }
    mt = wave64_max_dpp(mt);
    const float mn = fmaxf(m, mt);
    const float corr = (m == -INFINITY) ? 0.0f : __expf(m - mn);
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] *= corr;
    float ps = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const float p = t0 + kg + 8 * jj < j1 ? __expf(sc[jj] - mn) : 0.0f;
      ps += p;
#pragma unroll
      for (int e = 0; e < 8; e++) acc[e] += p * vr[jj].at(e);
    }
    // the tile's probability sum over the eight key groups (lane ^ 8, ^ 16, ^ 32)
    ps += dpp_pair<0x128>(ps);
    ps += swizzle_xor16(ps);
    ps += __shfl_xor(ps, 32, 64);
    l = l * corr + ps;
    m = mn;
  }
  __device__ __forceinline__ float finish() {
    const int lane = threadIdx.x & 63, dc = lane & 7;
    // add the eight key groups (lanes dc, dc + 8, .., dc + 56), then dimension `lane` sits
    // in element lane % 8 of lane lane / 8
#pragma unroll
    for (int e = 0; e < 8; e++) {
      acc[e] += dpp_pair<0x128>(acc[e]);  // row_ror:8 = lane ^ 8
      acc[e] += swizzle_xor16(acc[e]);
      acc[e] += __shfl_xor(acc[e], 32, 64);
    }
    float o = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x = __shfl(acc[e], lane >> 3, 64);
      if (dc == e) o = x;
    }
    return o;
  }
};

// One wave: attention of query q over keys j0..j1-1, the tiles' K and V rows loaded from
// the cache (all of a tile's loads in flight at once).  o returns dimension `lane`.
template <int KVT>
__device__ inline void attn_range(const float *q, const void *kh, const void *vh, int j0, int j1,
                                  float &m, float &l, float &o) {
  const int lane = threadIdx.x & 63, kg = lane >> 3, dc = lane & 7;
  AttnRun<KVT> run;
  run.init(q);
  for (int t0 = j0; t0 < j1; t0 += 64) {
    Row8<KVT> kr[8], vr[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int key = t0 + kg + 8 * jj;
      if (key < j1) {
        kr[jj].load(kh, (size_t)key, dc * 8);
        vr[jj].load(vh, (size_t)key, dc * 8);
      } else {
        kr[jj].zero();
        vr[jj].zero();
      }
    }
    run.tile(t0, j1, kr, vr);
  }
  o = run.finish();
  m = run.m;
  l = run.l;
}

struct AttnShared {
  float o[4][64];      // per-wave unnormalised outputs
  float m[4], l[4];
};

// One block of the decode attention: head h, key split s of the n_splits splits.  With
// WT, the partial is stored write-through (agent scope) for a combine in the same launch.
template <int KVT, bool WT = false>
__device__ inline void attn_decode_block(const float *q, const void *kc, const void *vc, int max_seq,
                                         const DecodeCtl *ctl, int static_len, float *part, int h, int s,
                                         int n_splits, AttnShared &sh) {
  const int L = ctl != nullptr ? ctl->valid_len + 1 : static_len;
  const int S = (L + kAttnKeys - 1) / kAttnKeys;  // active splits
  if (s >= S) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t hb = (size_t)h * max_seq * 64;
  const int jw = s * kAttnKeys + wave * 64;  // this wave's 64 keys (one tile of attn_range)
  float mw, lw, o;
  attn_range<KVT>(q + h * 64, head_base<KVT>(kc, hb), head_base<KVT>(vc, hb), jw, min(jw + 64, L), mw, lw, o);
  sh.o[wave][lane] = o;
  if (lane == 0) {
    sh.m[wave] = mw;
    sh.l[wave] = lw;
  }
  __syncthreads();
  // block partial: the four waves merged
  if (wave == 0) {
    float *mine = part + ((size_t)h * n_splits + s) * 66;
    float M = -INFINITY;
    for (int w = 0; w < 4; w++) M = fmaxf(M, sh.m[w]);
    float lsum = 0.0f, osum = 0.0f;
    for (int w = 0; w < 4; w++) {
      if (sh.m[w] == -INFINITY) continue;
      const float f = __expf(sh.m[w] - M);
      lsum += sh.l[w] * f;
      osum += sh.o[w][lane] * f;
    }
    if constexpr (WT) {
      __hip_atomic_store(reinterpret_cast<uint32_t *>(mine) + 2 + lane, __float_as_uint(osum), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 0) {
        __hip_atomic_store(reinterpret_cast<uint32_t *>(mine), __float_as_uint(M), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(reinterpret_cast<uint32_t *>(mine) + 1, __float_as_uint(lsum), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      mine[2 + lane] = osum;
      if (lane == 0) {
        mine[0] = M;
        mine[1] = lsum;
      }
    }
  }
}

template <int KVT>
__global__ __launch_bounds__(256) void attn_decode_kernel(const float *q, const void *kc, const void *vc,
                                                          int max_seq, const DecodeCtl *ctl, int static_len,
                                                          float *part) {
  if (ctl != nullptr && ctl->done) return;
  __shared__ AttnShared sh;
  attn_decode_block<KVT>(q, kc, vc, max_seq, ctl, static_len, part, blockIdx.x, blockIdx.y, gridDim.y, sh);
}

// One query row attended by the RW waves of a block over keys [0, L): wave w takes a
// contiguous run of the row's 64-key tiles (attn_range) and the runs are merged in LDS in
// wave order; no partials leave the block.  True in wave 0, whose lane holds dimension
// `lane` of the row's output in v; the other waves return false and leave.
template <int KVT, int RW>
__device__ __forceinline__ bool attn_row_merged(const float *q, const void *kh, const void *vh, int L, float &v) {
  __shared__ float so[RW][64], sm[RW], sl[RW];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = ((L + 63) / 64 + RW - 1) / RW;  // tiles per wave
  const int j0 = min(wave * per * 64, L), j1 = min((wave + 1) * per * 64, L);
  float m, l, o;
  attn_range<KVT>(q, kh, vh, j0, j1, m, l, o);
  so[wave][lane] = o;
  if (lane == 0) {
    sm[wave] = m;
    sl[wave] = l;
  }
  __syncthreads();
  if (wave != 0) return false;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < RW; w++) M = fmaxf(M, sm[w]);
  float den = 0.0f, num = 0.0f;
#pragma unroll
  for (int w = 0; w < RW; w++) {
    if (sm[w] == -INFINITY) continue;
    const float f = __expf(sm[w] - M);
    den += sl[w] * f;
    num += so[w][lane] * f;
  }
  v = num / den;
  return true;
}

// Batched decode attention, one block per (head, sequence): RW waves (16 for bf16 rows; 8
// for fp32 rows, whose tile registers would not fit 16 waves' 128 VGPRs) over the
// sequence's keys (attn_row_merged), into its attention row in the GEMM's split form.
template <int KVT>
constexpr int row_waves() {
  return KVT == kKvBf16 ? 16 : 8;
}
template <int KVT>
__global__ __launch_bounds__(64 * row_waves<KVT>()) void attn_decode_batch_row_kernel(const float *q,
                                                                                     const BatchSeq *seqs,
                                                                                     size_t layer_off, int max_seq,
                                                                                     SplitOut out) {
  const BatchSeq sq = seqs[blockIdx.y];
  if (sq.ctl->done) return;
  const int H = gridDim.x, d = H * 64, h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x & 63;
  const size_t es = KVT == kKvBf16 ? 2 : 4, hb = (size_t)h * max_seq * 64;
  const void *kc = static_cast<const char *>(sq.k) + layer_off * es;
  const void *vc = static_cast<const char *>(sq.v) + layer_off * es;
  float v;
  if (!attn_row_merged<KVT, row_waves<KVT>()>(q + (size_t)b * d + h * 64, head_base<KVT>(kc, hb),
                                              head_base<KVT>(vc, hb), sq.ctl->valid_len + 1, v))
    return;
  uint32_t hi, lo;
  split_f16(v, hi, lo);
  const size_t i = (size_t)b * d + h * 64 + lane;
  out.hi[i] = (uint16_t)hi;
  out.lo[i] = (uint16_t)lo;
  const float gsum = wave64_sum_dpp(v);
  if (lane == 0) out.gs[(size_t)b * (d / 64) + h] = gsum;
}

// Row b of a batched step: mel_emb[tok] + mel_pos[pos] of sequence b (from its control block).
__global__ __launch_bounds__(256) void embed_batch_kernel(const BatchSeq *seqs, const float *mel_emb,
                                                          const float *mel_pos, int d, float *x) {
  const DecodeCtl *ctl = seqs[blockIdx.x].ctl;
  const float *me = mel_emb + (size_t)ctl->tok * d;
  const float *mp = mel_pos + (size_t)ctl->pos * d;
  for (int i = threadIdx.x; i < d; i += 256) x[(size_t)blockIdx.x * d + i] = me[i] + mp[i];
}

// After a batched step: every running sequence has one more cache row.
__global__ void advance_batch_kernel(const BatchSeq *seqs, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B && !seqs[b].ctl->done) seqs[b].ctl->valid_len += 1;
}

// Stores one fp32 value of a row in the GEMM's split form; the wave's 64 lanes hold one
// 64-column group, whose sum lane 0 stores.
__device__ inline void put_split(const SplitOut &o, size_t i, size_t gi, float v) {
  uint32_t h, l;
  split_f16(v, h, l);
  o.hi[i] = (uint16_t)h;
  o.lo[i] = (uint16_t)l;
  const float s = wave64_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) o.gs[gi] = s;
}

// Global -> LDS copies issued by hand (lane l's 16 bytes land at lds + 16 l, lds in M0):
// issued with the builtin, the compiler would wait for every copy in flight before each LDS
// read; here the kernel's own s_waitcnt counts them.  M0 is set before every copy.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void attn_dma16(const void *src, const void *lds) {
  // the destination is the same for the whole wave (the callers' addresses are uniform)
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

// Prefill attention with the key tiles shared: one block of kPrefillRows waves per (head,
// kPrefillRows consecutive rows), wave w on row 4g + w.  Each 64-key tile of K and V is
// copied into LDS once (double-buffered, the next tile's copies in flight during this
// tile) and read by every wave from there, where a wave per row would read it from L2 once
// per row.  The tile arithmetic is AttnRun's, on the same rows, so each row's result is the
// one attn_range gives.  Measured at a 235-row prefill: 2.15-2.19 -> 2.11-2.13 ms against a
// wave per (head, row) reading its keys itself; 8 rows a block no faster; a row's tiles
// over 2 or 4 waves merged in LDS (attn_row_merged) no faster or slower (2.36 -> 2.44 ms).
constexpr int kPrefillRows = 4;
template <int KVT>
__global__ __launch_bounds__(64 * kPrefillRows) void attn_prefill_tiles_kernel(const float *q, int T, int base,
                                                                               const void *kc, const void *vc,
                                                                               int max_seq, int d, SplitOut out) {
  constexpr int ES = KVT == kKvBf16 ? 2 : 4;         // bytes per element
  constexpr int RB = 64 * ES, TB = 64 * RB;          // bytes per cache row, per 64-key tile
  constexpr int PIECES = TB / 16 / (64 * kPrefillRows);  // 16-byte copies per thread per tile and matrix
  __shared__ __attribute__((aligned(16))) char kv_lds[2][2][TB];  // [buffer][K, V][tile]
  // groups in reverse order, so the longest key ranges are dispatched first
  const int h = blockIdx.x, g = gridDim.y - 1 - blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, kg = lane >> 3, dc = lane & 7;
  const int t = kPrefillRows * g + wave;
  const int tl = min(t, T - 1);  // a wave past the last row runs that row and stores nothing
  const int L = base + tl + 1, Lb = base + min(kPrefillRows * g + kPrefillRows, T);
  const size_t hb = (size_t)h * max_seq * 64;
  const char *kb = static_cast<const char *>(head_base<KVT>(kc, hb));
  const char *vb = static_cast<const char *>(head_base<KVT>(vc, hb));
  const int ntile = (Lb + 63) / 64;
  // tile i into buffer i & 1: piece p = j * (64 kPrefillRows) + threadIdx.x of each matrix,
  // rows past the cache's end read its last row (never used: those keys are past every row)
  auto copy = [&](int i) {
#pragma unroll
    for (int j = 0; j < PIECES; j++) {
      const int pc = j * 64 * kPrefillRows + (int)threadIdx.x, row = pc * 16 / RB;
      const size_t off = (size_t)min(64 * i + row, max_seq - 1) * RB + (pc * 16) % RB;
      const int dst = (j * 64 * kPrefillRows + wave * 64) * 16;  // the wave's 1 KB, uniform
      attn_dma16(kb + off, &kv_lds[i & 1][0][dst]);
      attn_dma16(vb + off, &kv_lds[i & 1][1][dst]);
    }
  };
  AttnRun<KVT> run;
  run.init(q + (size_t)tl * d + h * 64);
  copy(0);
  for (int i = 0; i < ntile; i++) {
    if (i + 1 < ntile) {
      copy(i + 1);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PIECES) : "memory");  // tile i's copies
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (64 * i < L) {  // wave-uniform: the row's keys reach this tile
      Row8<KVT> kr[8], vr[8];
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        const int r = kg + 8 * jj;
        if (64 * i + r < L) {
          const uint4 *pk = reinterpret_cast<const uint4 *>(&kv_lds[i & 1][0][r * RB + dc * 8 * ES]);
          const uint4 *pv = reinterpret_cast<const uint4 *>(&kv_lds[i & 1][1][r * RB + dc * 8 * ES]);
          if constexpr (KVT == kKvBf16) {
            const uint4 a = pk[0], b = pv[0];
            kr[jj].w[0] = a.x; kr[jj].w[1] = a.y; kr[jj].w[2] = a.z; kr[jj].w[3] = a.w;
            vr[jj].w[0] = b.x; vr[jj].w[1] = b.y; vr[jj].w[2] = b.z; vr[jj].w[3] = b.w;
          } else {
            const uint4 a0 = pk[0], a1 = pk[1], b0 = pv[0], b1 = pv[1];
            kr[jj].w[0] = a0.x; kr[jj].w[1] = a0.y; kr[jj].w[2] = a0.z; kr[jj].w[3] = a0.w;
            kr[jj].w[4] = a1.x; kr[jj].w[5] = a1.y; kr[jj].w[6] = a1.z; kr[jj].w[7] = a1.w;
            vr[jj].w[0] = b0.x; vr[jj].w[1] = b0.y; vr[jj].w[2] = b0.z; vr[jj].w[3] = b0.w;
            vr[jj].w[4] = b1.x; vr[jj].w[5] = b1.y; vr[jj].w[6] = b1.z; vr[jj].w[7] = b1.w;
          }
        } else {
          kr[jj].zero();
          vr[jj].zero();
        }
      }
      run.tile(64 * i, L, kr, vr);
    }
    __syncthreads();  // buffer i & 1 is refilled with tile i + 2 next
  }
  const float o = run.finish();
  if (t < T) put_split(out, (size_t)t * d + h * 64 + lane, (size_t)t * (d / 64) + h, o / run.l);
}

// Attention probe (replay, gpt.rs:391-422): softmax probabilities of head p.head for the
// query rows p.q0.. over the key columns [p.k0, p.k1) of the K/V [n_head][ld][64]; row t
// attends to keys kstart[t]..t.  One block per query row; the attention output itself is
// produced by the flash kernel.
template <int KVT>
__global__ __launch_bounds__(64) void attn_probe_kernel(const float *q, const void *kc, const void *vc, int ld,
                                                        const int *kstart, int d, AttnProbe pr) {
  const int h = pr.head, t = pr.q0 + blockIdx.x, lane = threadIdx.x, kg = lane >> 3, dc = lane & 7;
  const size_t hb = (size_t)h * ld * 64;
  const int j0 = kstart[t];
  const void *kh = head_base<KVT>(kc, hb);
  const float *qt = q + (size_t)t * d + h * 64;
  float m, l, o;
  attn_range<KVT>(qt, kh, head_base<KVT>(vc, hb), j0, t + 1, m, l, o);
  const float4 qa = reinterpret_cast<const float4 *>(qt)[2 * dc], qb = reinterpret_cast<const float4 *>(qt)[2 * dc + 1];
  const int w = pr.k1 - pr.k0;
  for (int c0 = 0; c0 < w; c0 += 64) {
    // the scores of columns c0 + kg + 8 jj exactly as attn_range formed them, then column
    // c0 + lane taken from lane 8 (lane % 8), element lane / 8
    Row8<KVT> kr[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int j = pr.k0 + c0 + kg + 8 * jj;
      if (j >= j0 && j <= t) kr[jj].load(kh, (size_t)j, dc * 8);
      else kr[jj].zero();
    }
    float p = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const float sj = row_score<KVT>(qa, qb, kr[jj]);
      const float x = __shfl(sj, (lane & 7) << 3, 64);
      if ((lane >> 3) == jj) p = x;
    }
    const int c = c0 + lane, j = pr.k0 + c;
    if (c >= w) continue;
    pr.out[(size_t)(t - pr.q0) * w + c] = (j >= j0 && j <= t) ? __expf(p - m) / l : 0.0f;
  }
}

// log p(code_r | row r) = x[code] - max - log(sum exp(x - max)) over one logits row.
__global__ __launch_bounds__(256) void log_softmax_pick_kernel(const float *logits, int V, const int *codes,
                                                               float *out) {
  __shared__ float red[8];
  const float *x = logits + (size_t)blockIdx.x * V;
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < V; i += 256) mx = fmaxf(mx, x[i]);
  mx = wave64_max_dpp(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = 0.0f;
  for (int i = threadIdx.x; i < V; i += 256) s += expf(x[i] - mx);
  s = wave64_sum_dpp(s);
  if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float tot = (red[4] + red[5]) + (red[6] + red[7]);
    out[blockIdx.x] = (x[codes[blockIdx.x]] - mx) - logf(tot);
  }
}

// ---------------------------------------------------------------------------------
// Prefill embeddings and LayerNorm rows
// ---------------------------------------------------------------------------------

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

// One wave per row for d = 256 * NV (NV <= 8): lane l holds columns 256 j + 4 l .. + 3 of
// pass j in registers (16-byte loads), the mean and variance are DPP wave sums (no LDS, no
// barrier), and the 16 lanes of a DPP row hold one 64-column group, whose sum they form
// with four DPP steps.  Same arithmetic as ln_rows_kernel (biased variance, eps 1e-5; with
// w2, a second LayerNorm), summed in a different order.
template <int NV>
__device__ __forceinline__ void ln_regs(float4 (&v)[NV], const float *w, const float *b, int d, int lane) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean = wave64_sum_dpp(s) / (float)d;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const float a0 = v[j].x - mean, a1 = v[j].y - mean, a2 = v[j].z - mean, a3 = v[j].w - mean;
    q += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
  }
  const float rstd = 1.0f / sqrtf(wave64_sum_dpp(q) / (float)d + 1e-5f);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const float4 wj = reinterpret_cast<const float4 *>(w)[64 * j + lane];
    const float4 bj = reinterpret_cast<const float4 *>(b)[64 * j + lane];
    v[j].x = (v[j].x - mean) * rstd * wj.x + bj.x;
    v[j].y = (v[j].y - mean) * rstd * wj.y + bj.y;
    v[j].z = (v[j].z - mean) * rstd * wj.z + bj.z;
    v[j].w = (v[j].w - mean) * rstd * wj.w + bj.w;
  }
}

template <int NV>
__global__ __launch_bounds__(256) void ln_rows_wave_kernel(const float *x, const float *w, const float *b,
                                                           const float *w2, const float *b2, int T, int d,
                                                           SplitOut y) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;  // whole waves leave together
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * d);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) v[j] = xr[64 * j + lane];
  ln_regs<NV>(v, w, b, d, lane);
  if (w2) ln_regs<NV>(v, w2, b2, d, lane);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const size_t i = (size_t)row * d + 256 * j + 4 * lane;
    uint32_t h01, l01, h23, l23;
    split_f16x2(v[j].x, v[j].y, h01, l01);
    split_f16x2(v[j].z, v[j].w, h23, l23);
    *reinterpret_cast<uint2 *>(y.hi + i) = make_uint2(h01, h23);
    *reinterpret_cast<uint2 *>(y.lo + i) = make_uint2(l01, l23);
    // group 4 j + lane / 16: the 16 lanes of this DPP row
    float g = (v[j].x + v[j].y) + (v[j].z + v[j].w);
    g += dpp_pair<0xB1>(g);
    g += dpp_pair<0x4E>(g);
    g += dpp_pair<0x141>(g);
    g += dpp_pair<0x140>(g);
    if ((lane & 15) == 0) y.gs[(size_t)row * (d / 64) + 4 * j + (lane >> 4)] = g;
  }
}

// d is a multiple of 64, so each wave's 64 consecutive columns are one group.  With w2
// set, a second LayerNorm follows (ln_f then final_norm before the head).
__global__ __launch_bounds__(256) void ln_rows_kernel(const float *x, const float *w, const float *b,
                                                      const float *w2, const float *b2, int d, SplitOut y) {
  extern __shared__ float smem[];
  float *red = smem + d;
  layernorm_to_lds<256>(x + (size_t)blockIdx.x * d, w, b, d, smem, red);
  if (w2) layernorm_lds_inplace<256>(smem, w2, b2, d, red);
  for (int i = threadIdx.x; i < d; i += 256)
    put_split(y, (size_t)blockIdx.x * d + i, (size_t)blockIdx.x * (d / 64) + i / 64, smem[i]);
}

}  // namespace

hipError_t launch_gemv(const GemvArgs &a, int bits, int ptype, int pro, int epi, int kvt,
                       hipStream_t s) {
  const int epc = bits == 8 ? 16 : 32;
  if (a.ql.K % kGroup != 0 || a.ql.K / epc > 64 * 8) return hipErrorInvalidValue;
  if (pro == kProEmbedLN && a.ctl == nullptr) return hipErrorInvalidValue;
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

int attn_decode_max_splits(int max_seq) { return (max_seq + kAttnKeys - 1) / kAttnKeys; }

hipError_t launch_decode_batch_rows(const float *q, const BatchSeq *seqs, int B, size_t layer_off, int n_head,
                                    int max_seq, const SplitOut &out, int kvt, hipStream_t s) {
  dim3 grid(n_head, B);
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL(attn_decode_batch_row_kernel<kKvBf16>, grid, dim3(64 * row_waves<kKvBf16>()), 0, s, q, seqs,
                       layer_off, max_seq, out);
  } else {
    hipLaunchKernelGGL(attn_decode_batch_row_kernel<kKvF32>, grid, dim3(64 * row_waves<kKvF32>()), 0, s, q, seqs,
                       layer_off, max_seq, out);
  }
  return hipGetLastError();
}

hipError_t launch_embed_batch(const BatchSeq *seqs, int B, const float *mel_emb, const float *mel_pos, int d, float *x,
                              hipStream_t s) {
  hipLaunchKernelGGL(embed_batch_kernel, dim3(B), dim3(256), 0, s, seqs, mel_emb, mel_pos, d, x);
  return hipGetLastError();
}

hipError_t launch_advance_batch(const BatchSeq *seqs, int B, hipStream_t s) {
  hipLaunchKernelGGL(advance_batch_kernel, dim3((B + 63) / 64), dim3(64), 0, s, seqs, B);
  return hipGetLastError();
}

hipError_t launch_attn_decode(const float *q, const void *kc, const void *vc, int n_head,
                              int max_seq, const DecodeCtl *ctl, int static_len, float *part,
                              int kvt, hipStream_t s) {
  dim3 grid(n_head, attn_decode_max_splits(max_seq));
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL(attn_decode_kernel<kKvBf16>, grid, dim3(256), 0, s, q, kc, vc, max_seq, ctl, static_len,
                       part);
  } else {
    hipLaunchKernelGGL(attn_decode_kernel<kKvF32>, grid, dim3(256), 0, s, q, kc, vc, max_seq, ctl, static_len,
                       part);
  }
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
                          const SplitOut &y, hipStream_t s, const float *w2, const float *b2) {
  if (d % 64 != 0) return hipErrorInvalidValue;
  const dim3 grid4((T + 3) / 4);
  switch (d % 256 == 0 ? d / 256 : 0) {  // one wave per row when d = 256 * (1..8)
    case 1: hipLaunchKernelGGL(ln_rows_wave_kernel<1>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 2: hipLaunchKernelGGL(ln_rows_wave_kernel<2>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 3: hipLaunchKernelGGL(ln_rows_wave_kernel<3>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 4: hipLaunchKernelGGL(ln_rows_wave_kernel<4>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 5: hipLaunchKernelGGL(ln_rows_wave_kernel<5>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 6: hipLaunchKernelGGL(ln_rows_wave_kernel<6>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 7: hipLaunchKernelGGL(ln_rows_wave_kernel<7>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    case 8: hipLaunchKernelGGL(ln_rows_wave_kernel<8>, grid4, dim3(256), 0, s, x, w, b, w2, b2, T, d, y); break;
    default:
      hipLaunchKernelGGL(ln_rows_kernel, dim3(T), dim3(256), sizeof(float) * (d + 8), s, x, w, b, w2, b2, d, y);
  }
  return hipGetLastError();
}

hipError_t launch_attn_prefill(const float *q, int T, int base, const void *kc, const void *vc,
                               int n_head, int max_seq, const SplitOut &out, int kvt, hipStream_t s) {
  const int d = n_head * 64;
  if (T <= 0) return hipSuccess;
  dim3 grid(n_head, (T + kPrefillRows - 1) / kPrefillRows);
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL(attn_prefill_tiles_kernel<kKvBf16>, grid, dim3(64 * kPrefillRows), 0, s, q, T, base, kc, vc,
                       max_seq, d, out);
  } else {
    hipLaunchKernelGGL(attn_prefill_tiles_kernel<kKvF32>, grid, dim3(64 * kPrefillRows), 0, s, q, T, base, kc, vc,
                       max_seq, d, out);
  }
  return hipGetLastError();
}

hipError_t launch_attn_probe(const float *q, int M, const int *kstart, const void *kc, const void *vc, int n_head,
                             const AttnProbe &p, int kvt, hipStream_t s) {
  if (p.head < 0 || p.head >= n_head || p.q0 < 0 || p.q0 >= M || p.k0 < 0 || p.k1 <= p.k0 || !p.out)
    return hipErrorInvalidValue;
  const int d = n_head * 64;
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL(attn_probe_kernel<kKvBf16>, dim3(M - p.q0), dim3(64), 0, s, q, kc, vc, M, kstart, d, p);
  } else {
    hipLaunchKernelGGL(attn_probe_kernel<kKvF32>, dim3(M - p.q0), dim3(64), 0, s, q, kc, vc, M, kstart, d, p);
  }
  return hipGetLastError();
}

hipError_t launch_log_softmax_pick(const float *logits, int R, int V, const int *codes, float *out, hipStream_t s) {
  hipLaunchKernelGGL(log_softmax_pick_kernel, dim3(R), dim3(256), 0, s, logits, V, codes, out);
  return hipGetLastError();
}

}  // namespace itts
