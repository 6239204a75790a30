// Stage-2 CFM DiT estimator kernels for gfx950 (crates/core/src/models/cfm.rs).
//
// The estimator's linears are plain fp32 GEMMs and run in rocBLAS; the kernels here are
// the parts around them, fused where a GEMM's output is consumed elementwise: the
// timestep frequency embedding, AdaLN over RMSNorm (one pass per row), non-causal
// attention with rope applied while K and Q are staged (no rotated copy in HBM), SwiGLU,
// WaveNet's gated activation and residual / skip accumulation, the final layer norm with
// its modulation, and the Euler / classifier-free-guidance update.  Activations are
// [B][T][C] row-major fp32.
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
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
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

// Non-causal attention (scaled_dot_product_attention, scale 0.125, no mask) of one head over
// T positions, rope(traditional) applied to Q and K as they are staged (cfm.rs:274-289).
// qkv [B][T][3d] (q | k | v column blocks), out [B][T][d].  Block: 64 queries of (b, h),
// 256 threads; thread (q, part) scores keys part*16.. of each 64-key tile and accumulates
// output dimensions part*16.. .  Online softmax in fp32.
constexpr int kAq = 64, kAk = 64, kLd = 68;  // LDS row stride keeps 16-byte alignment
__global__ __launch_bounds__(256) void cfm_attn_kernel(const float *qkv, int T, int d, float *out) {
  __shared__ __attribute__((aligned(16))) float Ks[kAk * kLd];
  __shared__ __attribute__((aligned(16))) float Vs[kAk * kLd];
  __shared__ __attribute__((aligned(16))) float Ps[kAq * kLd];
  const int b = blockIdx.z, h = blockIdx.y, q0 = blockIdx.x * kAq;
  const int tid = threadIdx.x, qi = tid >> 2, part = tid & 3;
  const int qpos = q0 + qi;
  const size_t ld = 3 * (size_t)d;
  const float *base = qkv + (size_t)b * T * ld;
  float q[kHd];
  {
    const int qp = qpos < T ? qpos : T - 1;
    const float *qr = base + (size_t)qp * ld + h * kHd;
#pragma unroll
    for (int k = 0; k < kHd / 2; k++) {
      const float a = (float)qp * rope_inv(k), c = cosf(a), s = sinf(a);
      const float x0 = qr[2 * k], x1 = qr[2 * k + 1];
      q[2 * k] = x0 * c - x1 * s;
      q[2 * k + 1] = x0 * s + x1 * c;
    }
  }
  float m = -INFINITY, l = 0.0f, o[16];
#pragma unroll
  for (int e = 0; e < 16; e++) o[e] = 0.0f;
  for (int k0 = 0; k0 < T; k0 += kAk) {
    __syncthreads();
    for (int idx = tid; idx < kAk * (kHd / 2); idx += 256) {
      const int j = idx / (kHd / 2), k = idx % (kHd / 2), kp = k0 + j;
      float k0v = 0.0f, k1v = 0.0f, v0 = 0.0f, v1 = 0.0f;
      if (kp < T) {
        const float *kr = base + (size_t)kp * ld + d + h * kHd;
        const float a = (float)kp * rope_inv(k), c = cosf(a), s = sinf(a);
        const float x0 = kr[2 * k], x1 = kr[2 * k + 1];
        k0v = x0 * c - x1 * s;
        k1v = x0 * s + x1 * c;
        v0 = kr[d + 2 * k];
        v1 = kr[d + 2 * k + 1];
      }
      Ks[j * kLd + 2 * k] = k0v;
      Ks[j * kLd + 2 * k + 1] = k1v;
      Vs[j * kLd + 2 * k] = v0;
      Vs[j * kLd + 2 * k + 1] = v1;
    }
    __syncthreads();
    float s[16], mt = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 16; jj++) {
      const int j = part * 16 + jj;
      const float *kr = Ks + j * kLd;
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < kHd; e += 4) {
        const float4 kv = *reinterpret_cast<const float4 *>(kr + e);
        acc += q[e] * kv.x;
        acc += q[e + 1] * kv.y;
        acc += q[e + 2] * kv.z;
        acc += q[e + 3] * kv.w;
      }
      s[jj] = k0 + j < T ? acc * 0.125f : -INFINITY;
      mt = fmaxf(mt, s[jj]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 1, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 2, 64));
    const float mn = fmaxf(m, mt);
    const float alpha = expf(m - mn);
    float ls = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 16; jj++) {
      const float p = expf(s[jj] - mn);
      ls += p;
      Ps[qi * kLd + part * 16 + jj] = p;
    }
    ls += __shfl_xor(ls, 1, 64);
    ls += __shfl_xor(ls, 2, 64);
    l = l * alpha + ls;
    m = mn;
#pragma unroll
    for (int e = 0; e < 16; e++) o[e] *= alpha;
    __syncthreads();
    const float *pr = Ps + qi * kLd;
    for (int j = 0; j < kAk; j++) {
      const float p = pr[j];
      const float *vr = Vs + j * kLd + part * 16;
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const float4 vv = *reinterpret_cast<const float4 *>(vr + e);
        o[e] += p * vv.x;
        o[e + 1] += p * vv.y;
        o[e + 2] += p * vv.z;
        o[e + 3] += p * vv.w;
      }
    }
  }
  if (qpos < T) {
    float *orow = out + ((size_t)b * T + qpos) * d + h * kHd + part * 16;
    const float inv = 1.0f / l;
#pragma unroll
    for (int e = 0; e < 16; e++) orow[e] = o[e] * inv;
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
  hipLaunchKernelGGL(adaln_kernel, dim3(R), dim3(256), 0, s, x, y, T, d, mod, ld_mod, norm_w);
  return hipGetLastError();
}
hipError_t cfm_final_norm(const float *x, float *y, int R, int T, int d, const float *mod, hipStream_t s) {
  hipLaunchKernelGGL(final_norm_kernel, dim3(R), dim3(256), 0, s, x, y, T, d, mod);
  return hipGetLastError();
}
hipError_t cfm_attention(const float *qkv, int B, int T, int d, int H, float *out, hipStream_t s) {
  if (d != H * kHd) return hipErrorInvalidValue;
  hipLaunchKernelGGL(cfm_attn_kernel, dim3((T + kAq - 1) / kAq, H, B), dim3(256), 0, s, qkv, T, d, out);
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
