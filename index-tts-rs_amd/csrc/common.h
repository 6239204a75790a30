// Shared definitions of libitts_hip: device-side weight descriptors, decode control
// block, number-format helpers and wavefront reductions for gfx950 (wave64).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace itts {

constexpr int kHeadDim = 64;
constexpr int kGroup = 64;
constexpr int kSeenWords = 129;  // SeenTokenBitSet: 129 u64 words cover ids 0..8255

enum ParamType : int { kParamF16 = 0, kParamF32 = 1 };
enum KvType : int { kKvBf16 = 0, kKvF32 = 1 };

// One QuantizedLinear as stored on the device.
//   codes : bits=8 uint8 [N][K]; bits=4 uint8 [N][K/2] (low nibble = even k)
//   params: per (row, 64-group) the pair (scale, bias): fp16x2 packed in a uint32
//           (scale in the low half) or float2, [N][K/64]
//   bias  : fp32 [N]
struct DevQL {
  const uint8_t *codes;
  const void *params;
  const float *bias;
  int N, K;
};

struct DevLayer {
  const float *ln1_w, *ln1_b, *ln2_w, *ln2_b;
  DevQL attn, proj, fc, mproj;
};

// Per-sequence decode state kept in device memory so that one captured step can be
// replayed for every token: the kernels read the token, its position and the cache
// length from here, and the sampler writes the next ones.
struct DecodeCtl {
  int32_t tok;        // Mel token fed to the next step
  int32_t pos;        // its Mel position index
  int32_t valid_len;  // KV rows written before the next step
  int32_t done;       // generation finished (STOP sampled or max_steps reached)
  int32_t n_codes;    // codes emitted so far
  int32_t step;       // sampling step index s
  int32_t min_codes;
  int32_t max_steps;
  int32_t n_prior;
  int32_t last_tok;   // last sampled token (STOP included)
  uint64_t rng;       // SamplerRng state
  uint64_t seen[kSeenWords];
  // Owned by the device: steps taken by the persistent decode kernel (the epoch base of
  // its exchange words).  Host writes of the control block stop before this field.
  int32_t xstep;
  int32_t pad_;
};

// Sampling parameters as the device sampler consumes them.
struct DevSampling {
  int32_t greedy;
  float inv_temp;     // 1 / temperature, rounded once on the host
  float top_p;
  int32_t top_k;      // effective k (1..n)
  float penalty;
  int32_t apply_penalty;
};

__host__ __device__ inline uint32_t next_pow2(uint32_t v) {
  uint32_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

__device__ inline float half_bits_to_float(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)h));
}

__device__ inline float bf16_bits_to_float(uint32_t b) { return __uint_as_float(b << 16); }

// IEEE operations that round on their own: never fused into an FMA with a neighbour
// (hipcc contracts a*b+c by default, including through the __f*_rn helpers).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}
__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
  return a / b;
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ inline uint32_t float_to_bf16_bits(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (x >> 16) | 0x40u;
  x += 0x7fffu + ((x >> 16) & 1u);
  return x >> 16;
}

// x -> fp16 pair (hi, lo) with x = hi + lo to ~2^-22 relative (lo absorbs the rounding
// of hi; values below the fp16 normal range keep an absolute error under 2^-25).  |x| is
// clamped to the fp16 range for hi, so activations must stay below 65504 in magnitude.
__device__ inline void split_f16(float x, uint32_t &hi, uint32_t &lo) {
  const _Float16 h = (_Float16)fminf(fmaxf(x, -65504.0f), 65504.0f);
  const _Float16 l = (_Float16)(x - (float)h);
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, l);
}

// split_f16 of a pair (a, b), packed: hi = (hi_a, hi_b), lo = (lo_a, lo_b), low half first.
// The same values as two split_f16 calls (both conversions round to nearest even), formed
// by one v_cvt_pk_f16_f32 per plane and a single v_med3_f32 clamp per value.
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2e __attribute__((ext_vector_type(2)));
__device__ inline void split_f16x2(float a, float b, uint32_t &hi, uint32_t &lo) {
  const f32x2e v = {a, b};
  const f32x2e c = {__builtin_amdgcn_fmed3f(a, -65504.0f, 65504.0f), __builtin_amdgcn_fmed3f(b, -65504.0f, 65504.0f)};
  const f16x2v h = __builtin_convertvector(c, f16x2v);
  const f16x2v l = __builtin_convertvector(v - __builtin_convertvector(h, f32x2e), f16x2v);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}

// (scale, bias) of one (row, group).
template <int PT>
__device__ inline float2 load_param(const void *params, size_t idx) {
  if constexpr (PT == kParamF16) {
    const uint32_t w = static_cast<const uint32_t *>(params)[idx];
    return make_float2(half_bits_to_float(w & 0xffffu), half_bits_to_float(w >> 16));
  } else {
    return static_cast<const float2 *>(params)[idx];
  }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Reductions over each 32-lane half of a wave (lanes 0-31 and 32-63), result in every lane
// of the half.  Every step pairs lane i with a partner that pairs back with i (xor 1 and
// xor 2 within a quad, the 8-lane and 16-lane mirrors, then lane i ^ 16), so both lanes of
// a pair form the same value (a + b == b + a) and the half ends with one bit-identical
// result.  Four steps are DPP moves (VALU, no LDS round trip) and the last a ds_swizzle,
// so independent reductions overlap instead of waiting on five LDS permutes each.  Every
// lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_pair(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float swizzle_xor16(float v) {
  // bitmask mode: and 0x1f, or 0, xor 0x10 within each group of 32 lanes
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
}
__device__ __forceinline__ float half32_max(float v) {
  v = fmaxf(v, dpp_pair<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_pair<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_pair<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_pair<0x140>(v));  // row_mirror
  return fmaxf(v, swizzle_xor16(v));
}
__device__ __forceinline__ float half32_sum(float v) {
  v += dpp_pair<0xB1>(v);
  v += dpp_pair<0x4E>(v);
  v += dpp_pair<0x141>(v);
  v += dpp_pair<0x140>(v);
  return v + swizzle_xor16(v);
}
// Whole-wave versions: the two half results combined as wave-uniform scalars.
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wave64_max_dpp(float v) {
  v = half32_max(v);
  return fmaxf(lane_value(v, 0), lane_value(v, 32));
}
__device__ __forceinline__ float wave64_sum_dpp(float v) {
  v = half32_sum(v);
  return lane_value(v, 0) + lane_value(v, 32);
}

// gelu_approximate (tanh form).
__device__ inline float gelu_tanh(float x) {
  const float x3 = x * x * x;
  const float inner = 0.7978845608028654f * (x + 0.044715f * x3);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// The same function through 0.5 x (1 + tanh u) = x / (1 + exp(-2u)): one v_exp_f32 (2^t,
// t = -2u log2 e) and one v_rcp_f32, each within about an ulp, instead of tanhf's
// polynomial and branches; free of the cancellation in 1 + tanh u for negative x.  At
// u -> -inf, 2^t -> inf and the result -> -0; at u -> +inf, -> x.
__device__ inline float gelu_tanh_exp(float x) {
  const float u = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * u));
}

// Sum over a block of NT threads; every thread receives the same value, formed in the
// same order on every block (deterministic).
template <int NT>
__device__ inline float block_sum(float v, float *red) {
  v = wave64_sum_dpp(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < NT / 64; i++) t += red[i];
  __syncthreads();
  return t;
}

// LayerNorm of x[n] (global) into xl[n] (LDS): biased variance, eps 1e-5.
template <int NT>
__device__ inline void layernorm_to_lds(const float *x, const float *w, const float *b, int n,
                                        float *xl, float *red) {
  float s = 0.0f;
  for (int i = threadIdx.x; i < n; i += NT) {
    const float v = x[i];
    xl[i] = v;
    s += v;
  }
  const float mean = block_sum<NT>(s, red) / (float)n;
  float q = 0.0f;
  for (int i = threadIdx.x; i < n; i += NT) {
    const float d = xl[i] - mean;
    q += d * d;
  }
  const float var = block_sum<NT>(q, red) / (float)n;
  const float rstd = 1.0f / sqrtf(var + 1e-5f);
  for (int i = threadIdx.x; i < n; i += NT) xl[i] = (xl[i] - mean) * rstd * w[i] + b[i];
  __syncthreads();
}

// LayerNorm of an LDS row x into the LDS row y.
template <int NT>
__device__ inline void layernorm_lds_inplace_to(const float *x, float *y, const float *w, const float *b, int n,
                                                float *red) {
  float s = 0.0f;
  for (int i = threadIdx.x; i < n; i += NT) s += x[i];
  const float mean = block_sum<NT>(s, red) / (float)n;
  float q = 0.0f;
  for (int i = threadIdx.x; i < n; i += NT) {
    const float d = x[i] - mean;
    q += d * d;
  }
  const float var = block_sum<NT>(q, red) / (float)n;
  const float rstd = 1.0f / sqrtf(var + 1e-5f);
  for (int i = threadIdx.x; i < n; i += NT) y[i] = (x[i] - mean) * rstd * w[i] + b[i];
  __syncthreads();
}

// Same, in place on an LDS row.
template <int NT>
__device__ inline void layernorm_lds_inplace(float *xl, const float *w, const float *b, int n,
                                             float *red) {
  float s = 0.0f;
  for (int i = threadIdx.x; i < n; i += NT) s += xl[i];
  const float mean = block_sum<NT>(s, red) / (float)n;
  float q = 0.0f;
  for (int i = threadIdx.x; i < n; i += NT) {
    const float d = xl[i] - mean;
    q += d * d;
  }
  const float var = block_sum<NT>(q, red) / (float)n;
  const float rstd = 1.0f / sqrtf(var + 1e-5f);
  for (int i = threadIdx.x; i < n; i += NT) xl[i] = (xl[i] - mean) * rstd * w[i] + b[i];
  __syncthreads();
}

}  // namespace itts
