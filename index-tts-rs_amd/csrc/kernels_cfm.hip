// Stage-2 CFM DiT estimator kernels for gfx950 (crates/core/src/models/cfm.rs).
//
// The estimator's linears: the split-fp16 MFMA GEMM (fp32 operands split into fp16 hi/lo
// parts per K tile, fp32 accumulation) for products of 64 rows and more, and a few-row fp32
// FMA product (one wave per output column) for the per-batch conditioning projections and
// shorter forwards.  Around them, fused where a GEMM's output is consumed elementwise: the
// timestep frequency embedding, AdaLN over RMSNorm (one pass per row), non-causal MFMA
// attention (K with rope applied and V written once per call as fp16 hi/lo planes, Q
// rotated while staged), SwiGLU, WaveNet's gated activation and residual / skip
// accumulation, the final layer norm with its modulation, and the Euler /
// classifier-free-guidance update.  Activations are [B][T][C] row-major fp32.
#include "kernels.h"

namespace itts {

namespace {

constexpr int kHd = 64;          // head dimension (cfm.rs:42)
constexpr int kFreqHalf = 128;   // TimestepEmbedder: 128 frequencies (cfm.rs:115-121)

__device__ inline float silu(float x) { return x / (1.0f + expf(-x)); }
__device__ inline float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// Rope inverse frequency of pair k (compute_rope_freqs, cfm.rs:88-92).
__device__ inline float rope_inv(int k) { return 1.0f / powf(10000.0f, (float)(2 * k) / (float)kHd); }

// Block sum over 256 threads; red holds 8 floats.
__device__ inline float block_sum256(float v, float *red) {
  v = wave64_sum_dpp(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// emb[b] = [cos(t_b f_k), sin(t_b f_k)], f_k = 1000 exp(-ln(10000) k / 128) (cfm.rs:141-146)
__global__ void temb_kernel(const float *t, int B, float *emb) {
  const int b = blockIdx.x, k = threadIdx.x;
  if (b >= B || k >= kFreqHalf) return;
  const float f = 1000.0f * expf(-logf(10000.0f) * (float)k / (float)kFreqHalf);
  const float a = t[b] * f;
  emb[b * 2 * kFreqHalf + k] = cosf(a);
  emb[b * 2 * kFreqHalf + kFreqHalf + k] = sinf(a);
}

__global__ void silu_kernel(const float *x, float *y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = silu(x[i]);
}

// C[r][c] = bias[c] for r < rows, c < cols (rows ldc apart)
__global__ void bias_rows_kernel(float *C, int ldc, const float *bias, int rows, int cols) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * cols) return;
  const int r = (int)(i / cols), c = (int)(i % cols);
  C[(size_t)r * ldc + c] = bias[c];
}

// C[r][c] += bias[c]
__global__ void add_bias_kernel(float *C, int ldc, const float *bias, int rows, int cols) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * cols) return;
  const int r = (int)(i / cols), c = (int)(i % cols);
  C[(size_t)r * ldc + c] += bias[c];
}

// AdaLn::forward (cfm.rs:173-182) on row r = b*T + t: y = w_b * (x * rsqrt(mean(x^2) + 1e-5)
// * norm_w) + b_b, (w_b, b_b) = mod[b][0..d), mod[b][d..2d).  One 256-thread block per row.
__global__ __launch_bounds__(256) void adaln_kernel(const float *x, float *y, int T, int d, const float *mod,
                                                    int ld_mod, const float *norm_w) {
  __shared__ float red[8];
  const int r = blockIdx.x, b = r / T;
  const float *xr = x + (size_t)r * d;
  float s = 0.0f;
  for (int i = threadIdx.x; i < d; i += 256) s += xr[i] * xr[i];
  s = block_sum256(s, red);
  const float rs = 1.0f / sqrtf(s / (float)d + 1e-5f);
  const float *w = mod + (size_t)b * ld_mod, *bb = w + d;
  for (int i = threadIdx.x; i < d; i += 256) y[(size_t)r * d + i] = w[i] * (xr[i] * rs * norm_w[i]) + bb[i];
}

// adaln_kernel with one wave per row for d = 256 * NV: lane l holds columns 256 j + 4 l ..
// + 3 of pass j in registers, the mean square is a DPP wave sum (no LDS, no barrier).
template <int NV>
__global__ __launch_bounds__(256) void adaln_wave_kernel(const float *x, float *y, int R, int T, int d,
                                                         const float *mod, int ld_mod, const float *norm_w) {
  const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;  // whole waves leave together
  const int b = r / T;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)r * d);
  const float4 *w = reinterpret_cast<const float4 *>(mod + (size_t)b * ld_mod);
  const float4 *bb = reinterpret_cast<const float4 *>(mod + (size_t)b * ld_mod + d);
  const float4 *nw = reinterpret_cast<const float4 *>(norm_w);
  // the row, its batch's modulation and the norm weight all loaded before the reduction
  // (one memory round trip, not two)
  float4 v[NV], wv[NV], bv[NV], nv[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int c = 64 * j + lane;
    v[j] = xr[c];
    wv[j] = w[c];
    bv[j] = bb[c];
    nv[j] = nw[c];
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) s += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
  const float rs = 1.0f / sqrtf(wave64_sum_dpp(s) / (float)d + 1e-5f);
  float4 *yr = reinterpret_cast<float4 *>(y + (size_t)r * d);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int c = 64 * j + lane;
    const float4 wj = wv[j], bj = bv[j], nj = nv[j];
    yr[c] = make_float4(wj.x * (v[j].x * rs * nj.x) + bj.x, wj.y * (v[j].y * rs * nj.y) + bj.y,
                        wj.z * (v[j].z * rs * nj.z) + bj.z, wj.w * (v[j].w * rs * nj.w) + bj.w);
  }
}

// FinalLayer norm (cfm.rs:605-609): layer_norm(h, eps 1e-6, no affine) * (1 + scale_b) +
// shift_b, (shift_b, scale_b) = mod[b][0..d), mod[b][d..2d).
__global__ __launch_bounds__(256) void final_norm_kernel(const float *x, float *y, int T, int d, const float *mod) {
  __shared__ float red[8];
  const int r = blockIdx.x, b = r / T;
  const float *xr = x + (size_t)r * d;
  float s = 0.0f;
  for (int i = threadIdx.x; i < d; i += 256) s += xr[i];
  const float mean = block_sum256(s, red) / (float)d;
  float q = 0.0f;
  for (int i = threadIdx.x; i < d; i += 256) {
    const float v = xr[i] - mean;
    q += v * v;
  }
  q = block_sum256(q, red);
  const float rstd = 1.0f / sqrtf(q / (float)d + 1e-6f);
  const float *shift = mod + (size_t)b * 2 * d, *scale = shift + d;
  for (int i = threadIdx.x; i < d; i += 256)
    y[(size_t)r * d + i] = ((xr[i] - mean) * rstd) * (1.0f + scale[i]) + shift[i];
}

// Rope table (compute_rope_freqs, cfm.rs:73-101): tab[t][k] = (cos, sin) of t * inv_freq(k),
// k < 32, computed once per sequence length.
__global__ void rope_table_kernel(int T, float2 *tab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * (kHd / 2)) return;
  const int t = i / (kHd / 2), k = i % (kHd / 2);
  const float a = (float)t * rope_inv(k);
  tab[i] = make_float2(cosf(a), sinf(a));
}

// Non-causal attention on the MFMA units: scaled_dot_product_attention(scale 0.125, no mask)
// of one head over T positions, rope(traditional) applied to Q and K as they are staged
// (cfm.rs:274-289).  qkv [B][T][3d] (q | k | v column blocks) -> out [B][T][d].
//
// Block: two waves, 64 query rows of (head, batch); keys in tiles of 64.  Operands are split
// into fp16 hi/lo planes as they are staged, so S = Qh Kh + Qh Kl + Ql Kh and O += Ph Vh +
// Ph Vl + Pl Vh run on v_mfma_f32_32x32x16_f16 with ~22-bit operands and fp32 accumulation;
// online softmax in registers; P reaches the second product's operand layout through a
// per-wave LDS tile; 16-byte LDS chunks are XOR-swizzled by row.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
constexpr int kAq = 64, kAk = 64;

struct AttnLds {
  uint16_t k[2][kAk * 64];      // [plane][key][dim]
  uint16_t vt[2][64 * kAk];     // [plane][dim][key]
  uint16_t p[2][2][32 * kAk];   // [wave][plane][row][key]
};

// element offset of 16-byte chunk `chunk` of row `row` in a [row][64] fp16 array
__device__ __forceinline__ int swz(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3); }

__device__ __forceinline__ void split8(const float v[8], u32x4v &hi, u32x4v &lo) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t h, l;
    split_f16x2(v[2 * j], v[2 * j + 1], h, l);
    hi[j] = h;
    lo[j] = l;
  }
}

// 8 consecutive values of a head row at dims e0..e0+7 (e0 even), rotated for position t
__device__ __forceinline__ void load8_rope(const float *p, const float2 *tab, int t, int e0, float v[8]) {
  const float4 a = *reinterpret_cast<const float4 *>(p);
  const float4 b = *reinterpret_cast<const float4 *>(p + 4);
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const float2 *tr = tab + (size_t)t * (kHd / 2) + e0 / 2;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float2 cs = tr[j];
    v[2 * j] = x[2 * j] * cs.x - x[2 * j + 1] * cs.y;
    v[2 * j + 1] = x[2 * j] * cs.y + x[2 * j + 1] * cs.x;
  }
}

#define MFMA16 __builtin_amdgcn_mfma_f32_32x32x16_f16

// K (rope applied) and V of every (batch, head) as fp16 hi/lo planes, once per forward
// instead of once per query tile: K planes [B][H][Tp][64], V planes transposed [B][H][64][Tp]
// (keys contiguous), keys padded to Tp (a multiple of 64) with zeros.  ws holds the planes
// kh, kl, vh, vl of B * H * Tp * 64 values each.  The values are the ones the attention
// kernel formerly built while staging (same rope and split arithmetic).
__global__ __launch_bounds__(256) void kv_split_kernel(const float *qkv, const float2 *tab, int B, int T, int Tp, int d,
                                                       int H, uint16_t *ws) {
  const size_t plane = (size_t)B * H * Tp * kHd;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const long nk = (long)B * H * Tp * 8;  // K: one thread per (b, h, t, 8-dim chunk)
  const size_t ld3 = 3 * (size_t)d;
  if (i < nk) {
    const int c = (int)(i & 7);
    long r = i >> 3;
    const int t = (int)(r % Tp);
    r /= Tp;
    const int h = (int)(r % H), b = (int)(r / H);
    u32x4v hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
    if (t < T) {
      float v[8];
      load8_rope(qkv + ((size_t)b * T + t) * ld3 + d + h * kHd + c * 8, tab, t, c * 8, v);
      split8(v, hi, lo);
    }
    const size_t o = (((size_t)b * H + h) * Tp + t) * kHd + c * 8;
    *reinterpret_cast<u32x4v *>(ws + o) = hi;
    *reinterpret_cast<u32x4v *>(ws + plane + o) = lo;
    return;
  }
  // V: one thread per (b, h, 8-key chunk, dim), dim fastest (64 lanes read one row)
  const long j = i - nk, nkc = Tp / 8;
  if (j >= (long)B * H * nkc * kHd) return;
  const int e = (int)(j & 63);
  long r = j >> 6;
  const int kc = (int)(r % nkc);
  r /= nkc;
  const int h = (int)(r % H), b = (int)(r / H);
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int t = kc * 8 + k;
    v[k] = t < T ? qkv[((size_t)b * T + t) * ld3 + 2 * d + h * kHd + e] : 0.0f;
  }
  u32x4v hi, lo;
  split8(v, hi, lo);
  const size_t o = (((size_t)b * H + h) * kHd + e) * Tp + kc * 8;
  *reinterpret_cast<u32x4v *>(ws + 2 * plane + o) = hi;
  *reinterpret_cast<u32x4v *>(ws + 3 * plane + o) = lo;
}

// Keys are split over S blocks per query tile (blockIdx.z = b * S + split, kts key tiles
// each) so that short sequences still fill the chip; with S > 1 each block writes its
// unnormalised rows and their (max, denominator) to part_o [S][B][T][d] / part_ml
// [S][B][H][T][2], combined by attn_combine_kernel.
__global__ __launch_bounds__(128) void cfm_attn_kernel(const float *qkv, const float2 *tab, const uint16_t *kvs,
                                                       int Tp, int T, int d, int S, int kts, float *out,
                                                       float *part_o, float *part_ml) {
  __shared__ AttnLds sh;
  const int h = blockIdx.x, q0 = blockIdx.y * kAq, b = blockIdx.z / S, sp = blockIdx.z % S;
  const int B = gridDim.z / S, H = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const size_t ld3 = 3 * (size_t)d;
  const float *base = qkv + (size_t)b * T * ld3;
  // this (batch, head)'s planes from kv_split_kernel
  const size_t plane = (size_t)B * H * Tp * kHd, bh = (size_t)b * H + h;
  const uint16_t *kh_p = kvs + bh * Tp * kHd, *kl_p = kh_p + plane;
  const uint16_t *vh_p = kvs + 2 * plane + bh * kHd * Tp, *vl_p = vh_p + plane;

  // Q fragments of this lane's row (operand layout: row lane & 31, dims kk*16 + (lane>>5)*8 ..)
  f16x8 qh[4], ql[4];
  {
    const int t = min(q0 + w * 32 + (lane & 31), T - 1);
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const int e0 = kk * 16 + (lane >> 5) * 8;
      float v[8];
      load8_rope(base + (size_t)t * ld3 + h * kHd + e0, tab, t, e0, v);
      u32x4v hi, lo;
      split8(v, hi, lo);
      qh[kk] = __builtin_bit_cast(f16x8, hi);
      ql[kk] = __builtin_bit_cast(f16x8, lo);
    }
  }
  float m[16], l[16];
  floatx16 O[2];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
    O[0][i] = 0.0f;
    O[1][i] = 0.0f;
  }

  const int kend = min(T, (sp + 1) * kts * kAk);
  for (int kb = sp * kts * kAk; kb < kend; kb += kAk) {
    __syncthreads();  // the previous tile's operands are no longer read
    {  // K rows (rotated, split): thread -> key tid/2, 16-byte chunks (tid&1)*4 .. +3
      const int kr = tid >> 1;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int chunk = (tid & 1) * 4 + c;
        const size_t o = (size_t)(kb + kr) * kHd + chunk * 8;
        const u32x4v hi = *reinterpret_cast<const u32x4v *>(kh_p + o);
        const u32x4v lo = *reinterpret_cast<const u32x4v *>(kl_p + o);
        *reinterpret_cast<u32x4v *>(&sh.k[0][swz(kr, chunk)]) = hi;
        *reinterpret_cast<u32x4v *>(&sh.k[1][swz(kr, chunk)]) = lo;
      }
    }
    {  // V transposed: thread -> (dim e, 8-key chunk ck) for four of the 512 (e, ck) pairs
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int idx = tid * 4 + c, e = idx >> 3, ck = idx & 7;
        const size_t o = (size_t)e * Tp + kb + ck * 8;
        const u32x4v hi = *reinterpret_cast<const u32x4v *>(vh_p + o);
        const u32x4v lo = *reinterpret_cast<const u32x4v *>(vl_p + o);
        const int li = e * 64 + ((ck ^ ((e >> 1) & 7)) << 3);
        *reinterpret_cast<u32x4v *>(&sh.vt[0][li]) = hi;
        *reinterpret_cast<u32x4v *>(&sh.vt[1][li]) = lo;
      }
    }
    __syncthreads();

    floatx16 S[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int i = 0; i < 16; i++) S[kt][i] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const int o = swz(kt * 32 + (lane & 31), kk * 2 + (lane >> 5));
        const f16x8 bh = *reinterpret_cast<const f16x8 *>(&sh.k[0][o]);
        const f16x8 bl = *reinterpret_cast<const f16x8 *>(&sh.k[1][o]);
        S[kt] = MFMA16(qh[kk], bh, S[kt], 0, 0, 0);
        S[kt] = MFMA16(qh[kk], bl, S[kt], 0, 0, 0);
        S[kt] = MFMA16(ql[kk], bh, S[kt], 0, 0, 0);
      }
    }

    // masked, scaled scores and the 16 row maxima of the tile (independent reductions,
    // issued together)
    float tmax[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        const int key = kb + kt * 32 + (lane & 31);
        S[kt][i] = key >= T ? -INFINITY : S[kt][i] * 0.125f;
      }
      tmax[i] = half32_max(fmaxf(S[0][i], S[1][i]));
    }
    uint16_t *pw = sh.p[w][0];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float s[2] = {S[0][i], S[1][i]};
      const float mn = fmaxf(m[i], tmax[i]);
      // (__expf: v_exp_f32 on a pre-scaled argument, within a few ulp; the scores' own
      // rounding is far larger)
      const float corr = m[i] == -INFINITY ? 1.0f : __expf(m[i] - mn);
      const int r = (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      float psum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        const float p = s[kt] == -INFINITY ? 0.0f : __expf(s[kt] - mn);
        psum += p;
        uint32_t ph, pl;
        split_f16(p, ph, pl);
        const int key = kt * 32 + (lane & 31);
        const int o = r * 64 + (((key >> 3) ^ ((r >> 1) & 7)) << 3) + (key & 7);
        pw[o] = (uint16_t)ph;
        pw[32 * kAk + o] = (uint16_t)pl;
      }
      l[i] = l[i] * corr + psum;
      O[0][i] *= corr;
      O[1][i] *= corr;
      m[i] = mn;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's P tile is in LDS

#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const int oa = swz(lane & 31, kk * 2 + (lane >> 5));
      const f16x8 ah = *reinterpret_cast<const f16x8 *>(&pw[oa]);
      const f16x8 al = *reinterpret_cast<const f16x8 *>(&pw[32 * kAk + oa]);
#pragma unroll
      for (int dt = 0; dt < 2; dt++) {
        const int ob = swz(dt * 32 + (lane & 31), kk * 2 + (lane >> 5));
        const f16x8 bh = *reinterpret_cast<const f16x8 *>(&sh.vt[0][ob]);
        const f16x8 bl = *reinterpret_cast<const f16x8 *>(&sh.vt[1][ob]);
        O[dt] = MFMA16(ah, bh, O[dt], 0, 0, 0);
        O[dt] = MFMA16(ah, bl, O[dt], 0, 0, 0);
        O[dt] = MFMA16(al, bh, O[dt], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int t = q0 + w * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
    const float lt = half32_sum(l[i]);
    if (t < T) {
      if (S == 1) {
        float *orow = out + ((size_t)b * T + t) * d + h * kHd + (lane & 31);
        const float inv = 1.0f / lt;
        orow[0] = O[0][i] * inv;
        orow[32] = O[1][i] * inv;
      } else {
        float *orow = part_o + (((size_t)sp * B + b) * T + t) * d + h * kHd + (lane & 31);
        orow[0] = O[0][i];
        orow[32] = O[1][i];
        if ((lane & 31) == 0) {
          float *ml = part_ml + ((((size_t)sp * B + b) * H + h) * T + t) * 2;
          ml[0] = m[i];
          ml[1] = lt;
        }
      }
    }
  }
}

// Combines the key splits of cfm_attn_kernel: out = sum_s e^{m_s - M} O_s / sum_s e^{m_s - M} l_s.
// Every split's (m, l, O) is loaded before the first use (S <= kMaxSplits), so the loads
// take one round trip; the arithmetic and its order are those of a plain loop over s.
__global__ void attn_combine_kernel(const float *part_o, const float *part_ml, int S, int B, int T, int d,
                                    float *out) {
  constexpr int kMaxSplits = 8;  // cfm_attn_splits never returns more
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * T * d) return;
  const int c = (int)(i % d), bt = (int)(i / d), b = bt / T, t = bt % T, h = c / kHd, H = d / kHd;
  float mv[kMaxSplits], lv[kMaxSplits], ov[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++)
    if (s < S) {
      const float *ml = part_ml + ((((size_t)s * B + b) * H + h) * T + t) * 2;
      mv[s] = ml[0];
      lv[s] = ml[1];
      ov[s] = part_o[((size_t)s * B + b) * T * d + (size_t)t * d + c];
    }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++)
    if (s < S) M = fmaxf(M, mv[s]);
  float num = 0.0f, den = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++)
    if (s < S) {
      const float f = mv[s] == -INFINITY ? 0.0f : __expf(mv[s] - M);
      num += ov[s] * f;
      den += lv[s] * f;
    }
  out[i] = num / den;
}

// y[z][M][N] = A[z][M][K] W[z][N][K]^T + beta y on the MFMA units (the estimator's fp32
// Linear and conv layers, cfm.rs:200-411).  Operands are split into fp16 hi/lo planes as
// they are staged, y = Ah Wh + Ah Wl + Al Wh with fp32 accumulation (~22-bit operands, as
// in the attention above).  Block: 8 waves, a 64 x 64 tile of y; waves w and w + 4 share
// the 32 x 32 quarter w on v_mfma_f32_32x32x16_f16, each taking half of every K tile (two
// waves per SIMD even when the tiles only cover the chip once), their sums added through
// LDS at the end in a fixed order.  K in tiles of 64, double-buffered in LDS ([plane][row][k]
// with 16-byte chunks XOR-swizzled by row), the next tile's fp32 loads in flight while the
// MFMA units work on the current one: one barrier per K tile.  Rows of A may overlap (lda < K):
// a kernel-size-k conv over rows d apart is one GEMM with K = k d and lda = d.
// Requires K, lda, ldw % 4 == 0 and 16-byte aligned A and W.

struct GemmLds {
  uint16_t a[2][2][64 * 64];  // [buffer][plane][row][k]
  uint16_t w[2][2][64 * 64];
};

// W [N][ldw] (k < K) -> the pre-split quads split_gemm_kernel<true> reads, zeros past N and K.
// With ilv = F (N = 2F, the packed [w1; w3]), output row r holds input row (r >> 5 & 1) F +
// 32 (r >> 6) + (r & 31): each 64-row tile is 32 rows of w1 then the matching 32 of w3.
__global__ void split_weights_kernel(const float *W, int ldw, int N, int K, int kp4, long n, int ilv, uint4 *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int r = (int)(i / kp4), k = (int)(i % kp4) * 4;
  const int src = ilv ? ((r >> 5) & 1) * ilv + 32 * (r >> 6) + (r & 31) : r;
  uint4 q = make_uint4(0u, 0u, 0u, 0u);
  if (src < N && k < K) {
    const float4 v = *reinterpret_cast<const float4 *>(W + (size_t)src * ldw + k);
    split_f16x2(v.x, v.y, q.x, q.z);
    split_f16x2(v.z, v.w, q.y, q.w);
  }
  out[i] = q;
}

// W comes split already (cfm_split_weights): per row, 16 bytes per 4 values of k, {hi (k,
// k+1), hi (k+2, k+3), lo (k, k+1), lo (k+2, k+3)}, wkp4 quads a row, rows padded to a
// multiple of 64 and k to a multiple of 128 with zeros, copied to LDS as they are.
// SWIGLU (W split with ilv = F): tile columns 0-31 are w1 (gate) and 32-63 w3 (up) outputs
// of the same 32 columns of act = silu(gate) * up, written to y [M][ldy] (beta 0).
template <bool SWIGLU = false>
__global__ __launch_bounds__(512) void split_gemm_kernel(const float *A, int lda, long sa, const uint4 *Wp, int wkp4,
                                                         float *y, int ldy, long sy, int M, int N, int K, float beta,
                                                         const float *bias, const float *yr) {
  __shared__ GemmLds sh;
  const int tid = threadIdx.x, lane = tid & 63, wv = (tid >> 6) & 3, kg = tid >> 8, wm = wv >> 1, wn = wv & 1;
  const int n0 = blockIdx.x * 64, m0 = blockIdx.y * 64;
  A += blockIdx.z * sa;
  y += blockIdx.z * sy;
  const float *ysrc = yr ? yr + blockIdx.z * sy : y;  // beta's old values (y itself unless given)
  // K tiles of 64, rounded up to a pair (a tile past K is split as zeros), so that the
  // loop below runs whole pairs with no conditional step or store
  const int nk = (K + 127) / 128 * 2;
  // Two K tiles of fp32 loads in flight, in two register sets: a tile's loads are issued
  // two tiles before its split into LDS, so each waits behind a tile of MFMA work and a
  // barrier rather than being the next thing waited for (one set: each K tile cost about
  // one load latency).  The loads are unpredicated, with the row and k indexes clamped
  // into the operands (so that the compiler's wait counting keeps the later set in
  // flight).  Rows past M are loaded as a copy of the last row: they reach only output rows
  // that are not stored.  Values past K are zeros in W's planes (A's clamped values there
  // are finite, so the products vanish).
  float4 ra[2][2], rw[2][2];
  auto load = [&](int kt, float4(&a4)[2], float4(&w4)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int idx = tid + 512 * j, row = idx >> 4, k = min(kt * 64 + (idx & 15) * 4, K - 4);
      a4[j] = *reinterpret_cast<const float4 *>(A + (size_t)min(m0 + row, M - 1) * lda + k);
      w4[j] = __builtin_bit_cast(float4, Wp[(size_t)(n0 + row) * wkp4 + kt * 16 + (idx & 15)]);
    }
  };
  auto store = [&](int buf, int kt, const float4(&a4)[2], const float4(&w4)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int idx = tid + 512 * j, row = idx >> 4, c4 = idx & 15;
      const int off = swz(row, c4 >> 1) + (c4 & 1) * 4;
      const float4 av = a4[j];
      uint32_t ah0, al0, ah1, al1;
      split_f16x2(av.x, av.y, ah0, al0);
      split_f16x2(av.z, av.w, ah1, al1);
      const uint4 q = __builtin_bit_cast(uint4, w4[j]);
      const uint32_t wh0 = q.x, wh1 = q.y, wl0 = q.z, wl1 = q.w;
      *reinterpret_cast<uint2 *>(&sh.a[buf][0][off]) = make_uint2(ah0, ah1);
      *reinterpret_cast<uint2 *>(&sh.a[buf][1][off]) = make_uint2(al0, al1);
      *reinterpret_cast<uint2 *>(&sh.w[buf][0][off]) = make_uint2(wh0, wh1);
      *reinterpret_cast<uint2 *>(&sh.w[buf][1][off]) = make_uint2(wl0, wl1);
    }
  };
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.0f;
  // K tile kt: LDS buffer kt & 1; its registers set kt & 1, reloaded with tile kt + 2 once
  // the tile is in LDS.  Tiles past the end are loaded clamped; the last step's store
  // (tile nk, all zeros) goes to the buffer no later step reads.
  auto tile = [&](int kt, float4(&a_cur)[2], float4(&w_cur)[2], const float4(&a_nxt)[2],
                  const float4(&w_nxt)[2]) __attribute__((always_inline)) {
    const int buf = kt & 1;
    load(min(kt + 2, nk - 1), a_cur, w_cur);
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++) {
      const int kk = kg * 2 + k2;
      const int oa = swz(wm * 32 + (lane & 31), kk * 2 + (lane >> 5));
      const int ob = swz(wn * 32 + (lane & 31), kk * 2 + (lane >> 5));
      const f16x8 ah = *reinterpret_cast<const f16x8 *>(&sh.a[buf][0][oa]);
      const f16x8 al = *reinterpret_cast<const f16x8 *>(&sh.a[buf][1][oa]);
      const f16x8 bh = *reinterpret_cast<const f16x8 *>(&sh.w[buf][0][ob]);
      const f16x8 bl = *reinterpret_cast<const f16x8 *>(&sh.w[buf][1][ob]);
      acc = MFMA16(ah, bh, acc, 0, 0, 0);
      acc = MFMA16(ah, bl, acc, 0, 0, 0);
      acc = MFMA16(al, bh, acc, 0, 0, 0);
    }
    store(buf ^ 1, kt + 1, a_nxt, w_nxt);
    __syncthreads();
  };
  load(0, ra[0], rw[0]);
  load(min(1, nk - 1), ra[1], rw[1]);
  store(0, 0, ra[0], rw[0]);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    tile(kt, ra[0], rw[0], ra[1], rw[1]);
    tile(kt + 1, ra[1], rw[1], ra[0], rw[0]);
  }
  // the second K half's sums to LDS (the loop ended on a barrier), added by the first
  float *red = reinterpret_cast<float *>(&sh.a[0][0][0]) + wv * 1024 + lane;
  if (kg == 1) {
#pragma unroll
    for (int i = 0; i < 16; i++) red[i * 64] = acc[i];
  }
  __syncthreads();
  if constexpr (SWIGLU) {
    if (kg == 0) {
#pragma unroll
      for (int i = 0; i < 16; i++) acc[i] += red[i * 64];
    }
    __syncthreads();  // every read of red done before the area is reused
    float *up = reinterpret_cast<float *>(&sh.a[0][0][0]) + wm * 1024 + lane;
    if (kg == 0 && wn == 1) {
#pragma unroll
      for (int i = 0; i < 16; i++) up[i * 64] = acc[i];
    }
    __syncthreads();
    if (kg == 0 && wn == 0) {
      const int rb = m0 + wm * 32 + (lane >> 5) * 4, col = blockIdx.x * 32 + (lane & 31);
      float o[16];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        o[i] = silu(acc[i]) * up[i * 64];
        asm volatile("" : "+v"(o[i]));
      }
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int r = rb + (i >> 2) * 8 + (i & 3);
        if (r < M) y[(size_t)r * ldy + col] = o[i];
      }
    }
    return;
  }
  const int c = n0 + wn * 32 + (lane & 31);
  if (kg == 1 || c >= N) return;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] += red[i * 64];
  if (bias) {
    const float bc = bias[c];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = acc[i] + bc;
  }
  // With beta, the old outputs are loaded together (rows clamped, not predicated) and the
  // new values formed before the row-predicated stores: read and written element by
  // element, each load would wait behind the previous element's store.
  const int rb = m0 + wm * 32 + (lane >> 5) * 4;  // row of element 0
  if (beta != 0.0f) {
    float old[16];
#pragma unroll
    for (int i = 0; i < 16; i++) old[i] = ysrc[(size_t)min(rb + (i >> 2) * 8 + (i & 3), M - 1) * ldy + c];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      acc[i] = acc[i] + beta * old[i];
      asm volatile("" : "+v"(acc[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int r = rb + (i >> 2) * 8 + (i & 3);
    if (r < M) y[(size_t)r * ldy + c] = acc[i];
  }
}

// SwiGLU (cfm.rs:306-311): out[r][i] = silu(gu[r][i]) * gu[r][F + i]
__global__ void swiglu_kernel(const float *gu, int R, int F, float *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)R * F) return;
  const int r = (int)(i / F), c = (int)(i % F);
  out[i] = silu(gu[(size_t)r * 2 * F + c]) * gu[(size_t)r * 2 * F + F + c];
}

// WaveNet gated activation (cfm.rs:379-391): acts = conv + in_b + g_b; act = tanh(acts[:d]) *
// sigmoid(acts[d:]); g rows ld_g apart per batch.
__global__ void gate_kernel(const float *acts, const float *in_b, const float *g, int ld_g, int R, int T, int d,
                            float *act) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)R * d) return;
  const int r = (int)(i / d), c = (int)(i % d), b = r / T;
  const float *ar = acts + (size_t)r * 2 * d, *gb = g + (size_t)b * ld_g;
  const float a = ar[c] + in_b[c] + gb[c];
  const float s = ar[d + c] + in_b[d + c] + gb[d + c];
  act[i] = tanhf(a) * sigm(s);
}

// WaveNet residual / skip (cfm.rs:392-405): rs rows of width rso (+ rs_b); not last: h +=
// rs[:d], out += rs[d:]; last: out += rs.  h is the zero-padded [B][T + 2 pad][d] buffer.
__global__ void res_skip_kernel(const float *rs, const float *rs_b, int last, int R, int T, int d, int pad, float *h,
                                float *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)R * d) return;
  const int r = (int)(i / d), c = (int)(i % d), b = r / T, t = r % T;
  if (last) {
    out[i] += rs[(size_t)r * d + c] + rs_b[c];
  } else {
    h[((size_t)b * (T + 2 * pad) + t + pad) * d + c] += rs[(size_t)r * 2 * d + c] + rs_b[c];
    out[i] += rs[(size_t)r * 2 * d + d + c] + rs_b[d + c];
  }
}

// Euler step input (cfm.rs:727-731): x = x * mask (zero over the first T_ref frames); x_t =
// [x, x] transposed to [2][T][C], also the first C columns of both merged rows.
__global__ void euler_prep_kernel(float *x, int C, int T, int T_ref, float *xt, float *merged, int MD) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * T) return;
  const int c = (int)(i / T), t = (int)(i % T);
  float v = x[i];
  if (t < T_ref) {
    v = v * 0.0f;
    x[i] = v;
  }
  for (int b = 0; b < 2; b++) {
    xt[((size_t)b * T + t) * C + c] = v;
    merged[((size_t)b * T + t) * MD + c] = v;
  }
}

// Euler update with guidance (cfm.rs:735-745): x += dt * (pos * (1 + cfg) - neg * cfg), or dt *
// pos when cfg <= 0; v [2][T][C].
__global__ void euler_update_kernel(float *x, const float *v, int C, int T, float dt, float cfg) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * T) return;
  const int c = (int)(i / T), t = (int)(i % T);
  const float pos = v[(size_t)t * C + c], neg = v[((size_t)T + t) * C + c];
  const float g = cfg > 0.0f ? pos * (1.0f + cfg) - neg * cfg : pos;
  x[i] = x[i] + g * dt;
}

// Static CFG tail of the merged input (cfm.rs:682-711): columns [C, 2C) = prompt mel (row 0,
// frames < T_ref), [2C + d, 2C + d + S) = style (row 0); zeros elsewhere (pre-cleared).
__global__ void static_tail_kernel(float *merged, int MD, int C, int d, int S, int T, const float *ref_mel, int T_ref,
                                   const float *style) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)T * (C + S)) return;
  const int t = (int)(i / (C + S)), j = (int)(i % (C + S));
  float *row = merged + (size_t)t * MD;  // batch row 0
  if (j < C) {
    if (t < T_ref) row[C + j] = ref_mel[(size_t)j * T_ref + t];
  } else {
    row[2 * C + d + (j - C)] = style[j - C];
  }
}

// v [B][T][C] -> out [B][C][T]
__global__ void transpose_tc_kernel(const float *v, int B, int T, int C, float *out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * T * C) return;
  const int b = (int)(i / ((long)T * C)), rem = (int)(i % ((long)T * C)), t = rem / C, c = rem % C;
  out[((size_t)b * C + c) * T + t] = v[i];
}

// interior rows of the zero-padded WaveNet buffer from x [B][T][d]; the pad rows are zeroed
__global__ void pad_rows_kernel(const float *x, int B, int T, int d, int pad, float *hp) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int Tp = T + 2 * pad;
  if (i >= (long)B * Tp * d) return;
  const int b = (int)(i / ((long)Tp * d)), rem = (int)(i % ((long)Tp * d)), tp = rem / d, c = rem % d;
  const int t = tp - pad;
  hp[i] = (t >= 0 && t < T) ? x[((size_t)b * T + t) * d + c] : 0.0f;
}

// Few-row product y[z][m][n] = sum_k A[z][m][k] W[z][n][k] + beta y[z][m][n] in fp32 FMAs:
// the per-batch timestep / AdaLN / WaveNet-conditioning projections (2 rows, the CFG pair)
// and forwards of fewer than 64 rows.  One wave per output column n streams W's row n once
// (coalesced, VEC floats per lane) against MT rows of A (L2-resident); lane partial sums
// meet in a DPP reduction.  Block: 4 waves = 4 columns; grid (N/4, M/MT, batch).
template <int MT, int VEC>
__global__ __launch_bounds__(256) void rows_gemm_kernel(const float *__restrict__ A, int lda, long sa,
                                                        const float *__restrict__ W, int ldw, long sw, float *y,
                                                        int ldy, long sy, int M, int N, int K, float beta,
                                                        const float *bias, const float *yr) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int m0 = blockIdx.y * MT, z = blockIdx.z;
  const float *w = W + z * sw + (size_t)n * ldw;
  const float *a[MT];
#pragma unroll
  for (int j = 0; j < MT; j++) a[j] = A + z * sa + (size_t)(m0 + j < M ? m0 + j : m0) * lda;
  float acc[MT];
#pragma unroll
  for (int j = 0; j < MT; j++) acc[j] = 0.0f;
  if constexpr (VEC == 4) {
    for (int k = 4 * lane; k < K; k += 256) {
      const float4 wv = *reinterpret_cast<const float4 *>(w + k);
#pragma unroll
      for (int j = 0; j < MT; j++) {
        const float4 av = *reinterpret_cast<const float4 *>(a[j] + k);
        acc[j] = fmaf(av.x, wv.x, acc[j]);
        acc[j] = fmaf(av.y, wv.y, acc[j]);
        acc[j] = fmaf(av.z, wv.z, acc[j]);
        acc[j] = fmaf(av.w, wv.w, acc[j]);
      }
    }
  } else {
    for (int k = lane; k < K; k += 64) {
      const float wv = w[k];
#pragma unroll
      for (int j = 0; j < MT; j++) acc[j] = fmaf(a[j][k], wv, acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < MT; j++) acc[j] = wave64_sum_dpp(acc[j]);
  if (lane < MT && m0 + lane < M) {
    float v = acc[0];
#pragma unroll
    for (int j = 1; j < MT; j++)
      if (lane == j) v = acc[j];
    float *dst = y + z * sy + (size_t)(m0 + lane) * ldy + n;
    const float *src = yr ? yr + z * sy + (size_t)(m0 + lane) * ldy + n : dst;
    if (bias) v = v + bias[n];
    *dst = beta != 0.0f ? v + beta * *src : v;
  }
}

__global__ void fill_kernel(float *p, int n, float v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

inline unsigned nblk(long n, int t = 256) { return (unsigned)((n + t - 1) / t); }

}  // namespace

hipError_t cfm_temb(const float *t, int B, float *emb, hipStream_t s) {
  hipLaunchKernelGGL(temb_kernel, dim3(B), dim3(kFreqHalf), 0, s, t, B, emb);
  return hipGetLastError();
}
hipError_t cfm_silu(const float *x, float *y, int n, hipStream_t s) {
  hipLaunchKernelGGL(silu_kernel, dim3(nblk(n)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}
hipError_t cfm_bias_rows(float *C, int ldc, const float *bias, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(bias_rows_kernel, dim3(nblk((long)rows * cols)), dim3(256), 0, s, C, ldc, bias, rows, cols);
  return hipGetLastError();
}
hipError_t cfm_add_bias(float *C, int ldc, const float *bias, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(add_bias_kernel, dim3(nblk((long)rows * cols)), dim3(256), 0, s, C, ldc, bias, rows, cols);
  return hipGetLastError();
}
hipError_t cfm_adaln(const float *x, float *y, int R, int T, int d, const float *mod, int ld_mod, const float *norm_w,
                     hipStream_t s) {
  // one wave per row when d = 256 or 512 and the modulation rows keep 16-byte alignment
  const bool wave = (d == 256 || d == 512) && ld_mod % 4 == 0;
  if (wave && d == 512)
    hipLaunchKernelGGL(adaln_wave_kernel<2>, dim3((R + 3) / 4), dim3(256), 0, s, x, y, R, T, d, mod, ld_mod, norm_w);
  else if (wave)
    hipLaunchKernelGGL(adaln_wave_kernel<1>, dim3((R + 3) / 4), dim3(256), 0, s, x, y, R, T, d, mod, ld_mod, norm_w);
  else
    hipLaunchKernelGGL(adaln_kernel, dim3(R), dim3(256), 0, s, x, y, T, d, mod, ld_mod, norm_w);
  return hipGetLastError();
}
hipError_t cfm_final_norm(const float *x, float *y, int R, int T, int d, const float *mod, hipStream_t s) {
  hipLaunchKernelGGL(final_norm_kernel, dim3(R), dim3(256), 0, s, x, y, T, d, mod);
  return hipGetLastError();
}
hipError_t cfm_rope_table(int T, float *tab, hipStream_t s) {
  hipLaunchKernelGGL(rope_table_kernel, dim3(nblk((long)T * (kHd / 2))), dim3(256), 0, s, T,
                     reinterpret_cast<float2 *>(tab));
  return hipGetLastError();
}
int cfm_attn_splits(int B, int T, int H, int n_cu) {
  // The split with the fewest key tiles along the slowest block: rounds of blocks (three
  // resident per CU: 48 KB of LDS each) x key tiles per split, plus ~1.5 tiles' worth for
  // the combine pass when split.  (4 splits at 2 x 1033 rows: 1,088 blocks in two rounds of
  // 5 tiles; 5 splits: 1,360 blocks in two rounds of 4.)
  const int tiles = (T + kAk - 1) / kAk, blocks = H * ((T + kAq - 1) / kAq) * B;
  const int slots = 3 * (n_cu > 0 ? n_cu : 1);
  int bestS = 1;
  double best = 1e30;
  for (int S0 = 1; S0 <= 8 && S0 <= tiles; S0++) {
    const int kts = (tiles + S0 - 1) / S0, S = (tiles + kts - 1) / kts;  // no split without keys
    const int rounds = (blocks * S + slots - 1) / slots;
    const double cost = (double)rounds * kts + (S > 1 ? 1.5 : 0.0);
    if (cost < best) {
      best = cost;
      bestS = S;
    }
  }
  return bestS;
}
int cfm_kv_split_halves(int B, int T, int H) { return B * H * ((T + kAk - 1) / kAk) * kAk * kHd * 4; }

hipError_t cfm_attention(const float *qkv, const float *rope_tab, int B, int T, int d, int H, float *out,
                         float *part_o, float *part_ml, uint16_t *kv_split, int n_cu, hipStream_t s) {
  if (d != H * kHd || T < 1 || !kv_split) return hipErrorInvalidValue;
  const int S = cfm_attn_splits(B, T, H, n_cu), tiles = (T + kAk - 1) / kAk, kts = (tiles + S - 1) / S;
  if (S > 8 || (S > 1 && (!part_o || !part_ml))) return hipErrorInvalidValue;  // the combine holds 8
  const int Tp = tiles * kAk;
  const long nthreads = (long)B * H * Tp * 8 + (long)B * H * (Tp / 8) * kHd;
  hipLaunchKernelGGL(kv_split_kernel, dim3(nblk(nthreads)), dim3(256), 0, s, qkv,
                     reinterpret_cast<const float2 *>(rope_tab), B, T, Tp, d, H, kv_split);
  hipLaunchKernelGGL(cfm_attn_kernel, dim3(H, (T + kAq - 1) / kAq, B * S), dim3(128), 0, s, qkv,
                     reinterpret_cast<const float2 *>(rope_tab), kv_split, Tp, T, d, S, kts, out, part_o, part_ml);
  if (S > 1)
    hipLaunchKernelGGL(attn_combine_kernel, dim3(nblk((long)B * T * d)), dim3(256), 0, s, part_o, part_ml, S, B, T, d,
                       out);
  return hipGetLastError();
}
bool cfm_gemm_fits(const float *A, int lda, const float *W, int ldw, int K) {
  return K % 4 == 0 && lda % 4 == 0 && ldw % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(W) & 15) == 0;
}
size_t cfm_split_weights_quads(int N, int K) { return (size_t)((N + 63) / 64 * 64) * ((K + 127) / 128 * 32); }
hipError_t cfm_split_weights(const float *W, int ldw, int N, int K, uint4 *out, hipStream_t s, int ilv) {
  if (N < 1 || K < 4 || K % 4 || ldw % 4 || ldw < K || (reinterpret_cast<uintptr_t>(W) & 15)) return hipErrorInvalidValue;
  if (ilv && (ilv % 32 || N != 2 * ilv)) return hipErrorInvalidValue;
  const int kp4 = (K + 127) / 128 * 32;
  const long n = (long)((N + 63) / 64 * 64) * kp4;
  hipLaunchKernelGGL(split_weights_kernel, dim3(nblk(n)), dim3(256), 0, s, W, ldw, N, K, kp4, n, ilv, out);
  return hipGetLastError();
}
hipError_t cfm_gemm_swiglu(int M, int F, int K, const float *A, int lda, const uint4 *Wp, float *act, int ldo,
                           hipStream_t s) {
  if (M < 1 || F < 32 || F % 32 || K < 4 || K % 4 || lda % 4 || ldo < F || (reinterpret_cast<uintptr_t>(A) & 15) ||
      !Wp)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(split_gemm_kernel<true>, dim3(2 * F / 64, (M + 63) / 64, 1), dim3(512), 0, s, A, lda, 0L, Wp,
                     (K + 127) / 128 * 32, act, ldo, 0L, M, 2 * F, K, 0.0f, nullptr, nullptr);
  return hipGetLastError();
}
hipError_t cfm_gemm_split_w(int batch, int M, int N, int K, const float *A, int lda, long sa, const uint4 *Wp,
                            float *y, int ldy, long sy, float beta, hipStream_t s, const float *bias,
                            const float *yr) {
  if (batch < 1 || M < 1 || N < 1 || K < 4 || K % 4 || lda % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || !Wp)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(split_gemm_kernel<false>, dim3((N + 63) / 64, (M + 63) / 64, batch), dim3(512), 0, s, A, lda, sa,
                     Wp, (K + 127) / 128 * 32, y, ldy, sy, M, N, K, beta, bias, yr);
  return hipGetLastError();
}
hipError_t cfm_rows_gemm(int batch, int M, int N, int K, const float *A, int lda, long sa, const float *W, int ldw,
                         long sw, float *y, int ldy, long sy, float beta, hipStream_t s, const float *bias,
                         const float *yr) {
  if (batch < 1 || M < 1 || N < 1 || K < 1 || lda < K || ldw < K || ldy < N) return hipErrorInvalidValue;
  const bool v4 = K % 4 == 0 && lda % 4 == 0 && ldw % 4 == 0 && sa % 4 == 0 && sw % 4 == 0 &&
                  (reinterpret_cast<uintptr_t>(A) & 15) == 0 && (reinterpret_cast<uintptr_t>(W) & 15) == 0;
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const dim3 grid((N + 3) / 4, (M + mt - 1) / mt, batch);
#define ROWS_GEMM(MT, VEC)                                                                                        hipLaunchKernelGGL((rows_gemm_kernel<MT, VEC>), grid, dim3(256), 0, s, A, lda, sa, W, ldw, sw, y, ldy, sy, M, N,                      K, beta, bias, yr)
  if (v4) {
    if (mt == 1) ROWS_GEMM(1, 4);
    else if (mt == 2) ROWS_GEMM(2, 4);
    else if (mt == 4) ROWS_GEMM(4, 4);
    else ROWS_GEMM(8, 4);
  } else {
    if (mt == 1) ROWS_GEMM(1, 1);
    else if (mt == 2) ROWS_GEMM(2, 1);
    else if (mt == 4) ROWS_GEMM(4, 1);
    else ROWS_GEMM(8, 1);
  }
#undef ROWS_GEMM
  return hipGetLastError();
}
hipError_t cfm_swiglu(const float *gu, int R, int F, float *out, hipStream_t s) {
  hipLaunchKernelGGL(swiglu_kernel, dim3(nblk((long)R * F)), dim3(256), 0, s, gu, R, F, out);
  return hipGetLastError();
}
hipError_t cfm_gate(const float *acts, const float *in_b, const float *g, int ld_g, int R, int T, int d, float *act,
                    hipStream_t s) {
  hipLaunchKernelGGL(gate_kernel, dim3(nblk((long)R * d)), dim3(256), 0, s, acts, in_b, g, ld_g, R, T, d, act);
  return hipGetLastError();
}
hipError_t cfm_res_skip(const float *rs, const float *rs_b, int last, int R, int T, int d, int pad, float *h,
                        float *out, hipStream_t s) {
  hipLaunchKernelGGL(res_skip_kernel, dim3(nblk((long)R * d)), dim3(256), 0, s, rs, rs_b, last, R, T, d, pad, h, out);
  return hipGetLastError();
}
hipError_t cfm_euler_prep(float *x, int C, int T, int T_ref, float *xt, float *merged, int MD, hipStream_t s) {
  hipLaunchKernelGGL(euler_prep_kernel, dim3(nblk((long)C * T)), dim3(256), 0, s, x, C, T, T_ref, xt, merged, MD);
  return hipGetLastError();
}
hipError_t cfm_euler_update(float *x, const float *v, int C, int T, float dt, float cfg, hipStream_t s) {
  hipLaunchKernelGGL(euler_update_kernel, dim3(nblk((long)C * T)), dim3(256), 0, s, x, v, C, T, dt, cfg);
  return hipGetLastError();
}
hipError_t cfm_static_tail(float *merged, int MD, int C, int d, int S, int T, const float *ref_mel, int T_ref,
                           const float *style, hipStream_t s) {
  hipLaunchKernelGGL(static_tail_kernel, dim3(nblk((long)T * (C + S))), dim3(256), 0, s, merged, MD, C, d, S, T,
                     ref_mel, T_ref, style);
  return hipGetLastError();
}
hipError_t cfm_transpose_tc(const float *v, int B, int T, int C, float *out, hipStream_t s) {
  hipLaunchKernelGGL(transpose_tc_kernel, dim3(nblk((long)B * T * C)), dim3(256), 0, s, v, B, T, C, out);
  return hipGetLastError();
}
hipError_t cfm_pad_rows(const float *x, int B, int T, int d, int pad, float *hp, hipStream_t s) {
  hipLaunchKernelGGL(pad_rows_kernel, dim3(nblk((long)B * (T + 2 * pad) * d)), dim3(256), 0, s, x, B, T, d, pad, hp);
  return hipGetLastError();
}
hipError_t cfm_fill(float *p, int n, float v, hipStream_t s) {
  hipLaunchKernelGGL(fill_kernel, dim3(nblk(n)), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace itts
