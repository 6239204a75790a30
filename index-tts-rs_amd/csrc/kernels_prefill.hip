// Prefill GEMM for gfx950 and the standalone dequantiser.
//
// The GEMM contracts M activation rows against the int8 (or int4) codes on the MFMA
// units (v_mfma_f32_32x32x16_bf16).  Codes 0..255 are exact in bf16, so the matrix
// cores see the true integer weights; the activations enter as a bf16 hi/lo pair
// (x = hi + lo, ~16 significant bits) and both halves are accumulated in fp32.  The
// MLX group affine is applied per 64-wide K group on the fp32 partial:
//   acc += s[n,g] * (sum_{k in g} x[m,k] q[n,k]) + b[n,g] * (sum_{k in g} x[m,k]).
// Tiles: 64(M) x 64(N) per 256-thread block, 2x2 waves of 32x32, K step = one group.
#include "kernels.h"

namespace itts {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 64, BN = 64, BK = 64;

__device__ inline uint32_t bf16_pair_from_bytes(uint32_t w, int sh) {
  // two consecutive codes (bits sh..sh+15 of w) -> packed bf16 pair (exact)
  const float lo = (float)((w >> sh) & 0xffu);
  const float hi = (float)((w >> (sh + 8)) & 0xffu);
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

template <int BITS, int PT, int EPI, int KVT>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As_hi[BM][BK + 8];
  __shared__ __attribute__((aligned(16))) uint16_t As_lo[BM][BK + 8];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[BN][BK + 16];
  __shared__ float xs[BM];
  __shared__ float2 prm[BN];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int wm = wave >> 1, wn = wave & 1;
  const int K = a.ql.K, N = a.ql.N, M = a.M, G = K / kGroup;

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.0f;

  const int lr = tid >> 2, lc = (tid & 3) * 16;  // tile loader: row, first column
  for (int g = 0; g < G; g++) {
    {  // activations: 16 values of row lr -> bf16 hi/lo + group sum
      const int m = m0 + lr;
      float v[16];
      if (m < M) {
        const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)m * K + (size_t)g * BK + lc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float4 f = src[i];
          v[4 * i] = f.x;
          v[4 * i + 1] = f.y;
          v[4 * i + 2] = f.z;
          v[4 * i + 3] = f.w;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = 0.0f;
      }
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) s += v[i];
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      if ((tid & 3) == 0) xs[lr] = s;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t hb = float_to_bf16_bits(v[i]);
        const float lo = v[i] - __uint_as_float(hb << 16);
        As_hi[lr][lc + i] = (uint16_t)hb;
        As_lo[lr][lc + i] = (uint16_t)float_to_bf16_bits(lo);
      }
    }
    {  // codes of row lr, 16 elements from column lc of this group
      const int n = n0 + lr;
      uint4 u = make_uint4(0, 0, 0, 0);
      if constexpr (BITS == 8) {
        if (n < N) u = *reinterpret_cast<const uint4 *>(a.ql.codes + (size_t)n * K + (size_t)g * BK + lc);
      } else {
        if (n < N) {
          const uint2 p = *reinterpret_cast<const uint2 *>(a.ql.codes + (size_t)n * (K / 2) +
                                                            (size_t)g * (BK / 2) + lc / 2);
          const uint32_t w2[2] = {p.x, p.y};
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 2; i++) {
            const uint32_t w = w2[i];
            o[2 * i] = (w & 0xfu) | ((w >> 4) & 0xfu) << 8 | ((w >> 8) & 0xfu) << 16 | ((w >> 12) & 0xfu) << 24;
            o[2 * i + 1] = ((w >> 16) & 0xfu) | ((w >> 20) & 0xfu) << 8 | ((w >> 24) & 0xfu) << 16 |
                           ((w >> 28) & 0xfu) << 24;
          }
          u = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
      *reinterpret_cast<uint4 *>(&Bs[lr][lc]) = u;
    }
    if (tid < BN) {
      const int n = n0 + tid;
      prm[tid] = n < N ? load_param<PT>(a.ql.params, (size_t)n * G + g) : make_float2(0.0f, 0.0f);
    }
    __syncthreads();

    floatx16 P;
#pragma unroll
    for (int i = 0; i < 16; i++) P[i] = 0.0f;
    const int arow = wm * 32 + (lane & 31);
    const int brow = wn * 32 + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      const int kof = kk * 16 + (lane >> 5) * 8;
      const bf16x8 ahi = *reinterpret_cast<const bf16x8 *>(&As_hi[arow][kof]);
      const bf16x8 alo = *reinterpret_cast<const bf16x8 *>(&As_lo[arow][kof]);
      const uint2 bq = *reinterpret_cast<const uint2 *>(&Bs[brow][kof]);
      u32x4 bw;
      bw[0] = bf16_pair_from_bytes(bq.x, 0);
      bw[1] = bf16_pair_from_bytes(bq.x, 16);
      bw[2] = bf16_pair_from_bytes(bq.y, 0);
      bw[3] = bf16_pair_from_bytes(bq.y, 16);
      const bf16x8 b = __builtin_bit_cast(bf16x8, bw);
      P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi, b, P, 0, 0, 0);
      P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo, b, P, 0, 0, 0);
    }
    const float2 sb = prm[wn * 32 + (lane & 31)];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = wm * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      acc[i] += sb.x * P[i] + sb.y * xs[r];
    }
    __syncthreads();
  }

  const int n = n0 + wn * 32 + (lane & 31);
  if (n >= N) return;
  const float bias = a.ql.bias[n];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int m = m0 + wm * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
    if (m >= M) continue;
    const float v = acc[i] + bias;
    if constexpr (EPI == kEpiStore) {
      a.y[(size_t)m * N + n] = v;
    } else if constexpr (EPI == kEpiResid) {
      a.y[(size_t)m * N + n] += v;
    } else if constexpr (EPI == kEpiGelu) {
      a.y[(size_t)m * N + n] = gelu_tanh(v);
    } else {
      const int d = a.qkv.d_model;
      if (n < d) {
        a.qkv.q_out[(size_t)m * d + n] = v;
      } else {
        const int idx = n < 2 * d ? n - d : n - 2 * d;
        const int h = idx >> 6, e = idx & 63;
        const size_t ci = ((size_t)h * a.qkv.max_seq + a.qkv.pos0 + m) * kHeadDim + e;
        void *cache = n < 2 * d ? a.qkv.k_cache : a.qkv.v_cache;
        if constexpr (KVT == kKvBf16) {
          static_cast<uint16_t *>(cache)[ci] = (uint16_t)float_to_bf16_bits(v);
        } else {
          static_cast<float *>(cache)[ci] = v;
        }
      }
    }
  }
}

template <int BITS, int PT>
hipError_t gemm_dispatch(const GemmArgs &a, int epi, int kvt, hipStream_t s) {
  dim3 grid((a.ql.N + BN - 1) / BN, (a.M + BM - 1) / BM);
  switch (epi) {
    case kEpiStore:
      hipLaunchKernelGGL((gemm_kernel<BITS, PT, kEpiStore, 0>), grid, dim3(256), 0, s, a);
      break;
    case kEpiResid:
      hipLaunchKernelGGL((gemm_kernel<BITS, PT, kEpiResid, 0>), grid, dim3(256), 0, s, a);
      break;
    case kEpiGelu:
      hipLaunchKernelGGL((gemm_kernel<BITS, PT, kEpiGelu, 0>), grid, dim3(256), 0, s, a);
      break;
    case kEpiQKV:
      if (kvt == kKvBf16) {
        hipLaunchKernelGGL((gemm_kernel<BITS, PT, kEpiQKV, kKvBf16>), grid, dim3(256), 0, s, a);
      } else {
        hipLaunchKernelGGL((gemm_kernel<BITS, PT, kEpiQKV, kKvF32>), grid, dim3(256), 0, s, a);
      }
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// out[o][k] = float(q) * s then + b: two roundings, no contraction.
template <int BITS, int PT>
__global__ __launch_bounds__(256) void dequant_kernel(DevQL ql, float *out) {
#pragma clang fp contract(off)
  const size_t total = (size_t)ql.N * ql.K;
  const int G = ql.K / kGroup;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const int o = (int)(i / ql.K), k = (int)(i % ql.K);
    int q;
    if constexpr (BITS == 8) {
      q = ql.codes[i];
    } else {
      const uint8_t b = ql.codes[(size_t)o * (ql.K / 2) + k / 2];
      q = (k & 1) ? (b >> 4) : (b & 0xf);
    }
    const float2 sb = load_param<PT>(ql.params, (size_t)o * G + k / kGroup);
    out[i] = add_rn(mul_rn((float)q, sb.x), sb.y);
  }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs &a, int bits, int ptype, int epi, int kvt, hipStream_t s) {
  if (a.ql.K % kGroup != 0 || a.M <= 0) return hipErrorInvalidValue;
  if (bits == 8) {
    return ptype == kParamF16 ? gemm_dispatch<8, kParamF16>(a, epi, kvt, s)
                              : gemm_dispatch<8, kParamF32>(a, epi, kvt, s);
  }
  if (bits == 4) {
    return ptype == kParamF16 ? gemm_dispatch<4, kParamF16>(a, epi, kvt, s)
                              : gemm_dispatch<4, kParamF32>(a, epi, kvt, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dequant(const DevQL &ql, int bits, int ptype, float *out, hipStream_t s) {
  const size_t total = (size_t)ql.N * ql.K;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 8192);
  if (bits == 8) {
    if (ptype == kParamF16) hipLaunchKernelGGL((dequant_kernel<8, kParamF16>), dim3(blocks), dim3(256), 0, s, ql, out);
    else hipLaunchKernelGGL((dequant_kernel<8, kParamF32>), dim3(blocks), dim3(256), 0, s, ql, out);
  } else if (bits == 4) {
    if (ptype == kParamF16) hipLaunchKernelGGL((dequant_kernel<4, kParamF16>), dim3(blocks), dim3(256), 0, s, ql, out);
    else hipLaunchKernelGGL((dequant_kernel<4, kParamF32>), dim3(blocks), dim3(256), 0, s, ql, out);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace itts
