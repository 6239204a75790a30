// Causal multi-row attention on the MFMA units (prefill, replay, all-row forward).
//
// Block: two waves, 64 query rows of one head (wave w owns rows 32w..32w+31 in the MFMA
// output layout).  Keys are processed in tiles of 64: the K rows and the transposed V
// rows of a tile are read from the cache (bf16 or fp32 [n_head][ld][64]) and split into
// fp16 hi/lo planes as they are staged in LDS, so that
//   S = Q K^T = Qh Kh + Qh Kl + Ql Kh      and      O += P V = Ph Vh + Ph Vl + Pl Vh
// run on v_mfma_f32_32x32x16_f16 with ~22-bit operands and fp32 accumulation.  The
// softmax is online (running row max and denominator in registers); P goes through a
// per-wave LDS tile to reach the operand layout of the second product.  16-byte LDS
// chunks are XOR-swizzled by (row >> 1) & 7 (a 128-byte row is half of gfx950's 256-byte
// bank row) so that fragment reads spread over the 64 banks.
//
// Query row t sits at cache position base + t and attends to keys ks(t)..base + t, with
// ks(t) = kstart[t] (concatenated sequences) or 0.
#include "kernels.h"

namespace itts {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kFQ = 64;  // query rows per block
constexpr int kFK = 64;  // keys per tile

struct FlashLds {
  uint16_t k[2][kFK * 64];      // [plane][key][dim]
  uint16_t vt[2][64 * kFK];     // [plane][dim][key]
  uint16_t p[2][2][32 * kFK];   // [wave][plane][row][key]
};

// element offset of 16-byte chunk `chunk` of row `row` in a [row][64] fp16 array
__device__ __forceinline__ int swz(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3); }

template <int KVT>
__device__ __forceinline__ void load8(const void *base, size_t idx, float v[8]) {
  if constexpr (KVT == kKvBf16) {
    const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + idx);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx);
    const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
}

__device__ __forceinline__ void split8(const float v[8], u32x4 &hi, u32x4 &lo) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t h, l;
    split_f16x2(v[2 * j], v[2 * j + 1], h, l);
    hi[j] = h;
    lo[j] = l;
  }
}

#define MFMA16 __builtin_amdgcn_mfma_f32_32x32x16_f16

// K and V of every head as fp16 hi/lo planes for keys 0..L-1, once per layer instead of
// once per query tile: K planes [H][Lp][64], V planes transposed [H][64][Lp] (keys
// contiguous), keys padded to Lp (a multiple of 64) with zeros.  ws holds kh, kl, vh, vl of
// H * Lp * 64 values each; the values are the ones the flash kernel otherwise builds while
// staging (same split).
template <int KVT>
__global__ __launch_bounds__(256) void kv_split_kernel(const void *kc, const void *vc, int ld, int H, int L, int Lp,
                                                       uint16_t *ws) {
  const size_t plane = (size_t)H * Lp * 64;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const long nk = (long)H * Lp * 8;  // K: one thread per (h, key, 8-dim chunk)
  if (i < nk) {
    const int c = (int)(i & 7);
    const long r = i >> 3;
    const int t = (int)(r % Lp), h = (int)(r / Lp);
    u32x4 hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
    if (t < L) {
      float v[8];
      load8<KVT>(kc, ((size_t)h * ld + t) * 64 + c * 8, v);
      split8(v, hi, lo);
    }
    const size_t o = ((size_t)h * Lp + t) * 64 + c * 8;
    *reinterpret_cast<u32x4 *>(ws + o) = hi;
    *reinterpret_cast<u32x4 *>(ws + plane + o) = lo;
    return;
  }
  // V: one thread per (h, 8-key chunk, dim), dim fastest (64 lanes read one row)
  const long j = i - nk, nkc = Lp / 8;
  if (j >= (long)H * nkc * 64) return;
  const int e = (int)(j & 63);
  const long r = j >> 6;
  const int kc8 = (int)(r % nkc), h = (int)(r / nkc);
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int t = kc8 * 8 + k;
    const size_t idx = ((size_t)h * ld + min(t, L - 1)) * 64 + e;
    const float x = KVT == kKvBf16 ? __uint_as_float((uint32_t) static_cast<const uint16_t *>(vc)[idx] << 16)
                                   : static_cast<const float *>(vc)[idx];
    v[k] = t < L ? x : 0.0f;
  }
  u32x4 hi, lo;
  split8(v, hi, lo);
  const size_t o = ((size_t)h * 64 + e) * Lp + kc8 * 8;
  *reinterpret_cast<u32x4 *>(ws + 2 * plane + o) = hi;
  *reinterpret_cast<u32x4 *>(ws + 3 * plane + o) = lo;
}

// PRE: K/V come from kv_split_kernel's planes (kvs, keys padded to Lp) and are staged by
// 16-byte copies; otherwise they are read from the cache and split while staged.
template <int KVT, bool PRE>
__global__ __launch_bounds__(128) void attn_flash_kernel(const float *q, int d, const void *kc, const void *vc,
                                                         int ld, int base, int T, const int *kstart, SplitOut out,
                                                         const uint16_t *kvs, int Lp, const int *order) {
  __shared__ FlashLds sh;
  const int h = blockIdx.x, q0 = (order ? order[blockIdx.y] : (int)blockIdx.y) * kFQ;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const size_t hb = (size_t)h * ld * 64;
  const void *kh = KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(kc) + hb)
                                  : (const void *)(static_cast<const float *>(kc) + hb);
  const void *vh = KVT == kKvBf16 ? (const void *)(static_cast<const uint16_t *>(vc) + hb)
                                  : (const void *)(static_cast<const float *>(vc) + hb);

  // Q fragments of this lane's row (operand layout: row lane & 31, dims kk*16 + (lane>>5)*8 ..)
  f16x8 qh[4], ql[4];
  {
    const int t = min(q0 + w * 32 + (lane & 31), T - 1);
    const float *qp = q + (size_t)t * d + h * 64 + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      float v[8];
      const float4 a = *reinterpret_cast<const float4 *>(qp + kk * 16);
      const float4 b = *reinterpret_cast<const float4 *>(qp + kk * 16 + 4);
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
      u32x4 hi, lo;
      split8(v, hi, lo);
      qh[kk] = __builtin_bit_cast(f16x8, hi);
      ql[kk] = __builtin_bit_cast(f16x8, lo);
    }
  }
  // output-layout rows of this lane: r(i) = (i>>2)*8 + (lane>>5)*4 + (i&3)
  int pos[16], ks[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int t = q0 + w * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
    pos[i] = base + t;
    ks[i] = kstart ? kstart[min(t, T - 1)] : 0;
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

  const int kmin = kstart ? kstart[q0] : 0;
  const int kmax = base + min(q0 + kFQ - 1, T - 1);
  for (int kb = (kmin / kFK) * kFK; kb <= kmax; kb += kFK) {
    __syncthreads();  // the previous tile's operands are no longer read
    if constexpr (PRE) {
      const size_t plane = (size_t)gridDim.x * Lp * 64;
      {  // K rows: thread -> key tid/2, 16-byte chunks (tid&1)*4 .. +3
        const int kr = tid >> 1;
        const uint16_t *khp = kvs + ((size_t)h * Lp + kb + kr) * 64;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int chunk = (tid & 1) * 4 + c;
          const u32x4 hi = *reinterpret_cast<const u32x4 *>(khp + chunk * 8);
          const u32x4 lo = *reinterpret_cast<const u32x4 *>(khp + plane + chunk * 8);
          *reinterpret_cast<u32x4 *>(&sh.k[0][swz(kr, chunk)]) = hi;
          *reinterpret_cast<u32x4 *>(&sh.k[1][swz(kr, chunk)]) = lo;
        }
      }
      {  // V transposed: thread -> (dim e, 8-key chunk ck) for four of the 512 pairs
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int idx = tid * 4 + c, e = idx >> 3, ck = idx & 7;
          const uint16_t *vp = kvs + 2 * plane + ((size_t)h * 64 + e) * Lp + kb + ck * 8;
          const u32x4 hi = *reinterpret_cast<const u32x4 *>(vp);
          const u32x4 lo = *reinterpret_cast<const u32x4 *>(vp + plane);
          const int li = e * 64 + ((ck ^ ((e >> 1) & 7)) << 3);
          *reinterpret_cast<u32x4 *>(&sh.vt[0][li]) = hi;
          *reinterpret_cast<u32x4 *>(&sh.vt[1][li]) = lo;
        }
      }
      __syncthreads();
    } else {
      {  // K rows: thread -> key tid/2, dims (tid&1)*32 .. +31
        const int kr = tid >> 1, key = min(kb + kr, ld - 1);
  #pragma unroll
        for (int c = 0; c < 4; c++) {
          const int chunk = (tid & 1) * 4 + c;
          float v[8];
          load8<KVT>(kh, (size_t)key * 64 + chunk * 8, v);
          u32x4 hi, lo;
          split8(v, hi, lo);
          *reinterpret_cast<u32x4 *>(&sh.k[0][swz(kr, chunk)]) = hi;
          *reinterpret_cast<u32x4 *>(&sh.k[1][swz(kr, chunk)]) = lo;
        }
      }
      {  // V transposed: thread -> keys 2kp, 2kp+1, dims (tid&3)*16 .. +15
        const int kp = tid >> 2;
        const int k0 = min(kb + 2 * kp, ld - 1), k1 = min(kb + 2 * kp + 1, ld - 1);
  #pragma unroll
        for (int c = 0; c < 2; c++) {
          const int e0 = (tid & 3) * 16 + c * 8;
          float a[8], b[8];
          load8<KVT>(vh, (size_t)k0 * 64 + e0, a);
          load8<KVT>(vh, (size_t)k1 * 64 + e0, b);
  #pragma unroll
          for (int j = 0; j < 8; j++) {
            const int e = e0 + j;
            uint32_t hab, lab;
            split_f16x2(a[j], b[j], hab, lab);
            const int idx = e * 64 + ((((2 * kp) >> 3) ^ ((e >> 1) & 7)) << 3) + ((2 * kp) & 7);
            *reinterpret_cast<uint32_t *>(&sh.vt[0][idx]) = hab;
            *reinterpret_cast<uint32_t *>(&sh.vt[1][idx]) = lab;
          }
        }
      }
      __syncthreads();
    }

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
        S[kt][i] = (key > pos[i] || key < ks[i]) ? -INFINITY : S[kt][i] * 0.125f;
      }
      tmax[i] = half32_max(fmaxf(S[0][i], S[1][i]));
    }
    uint16_t *pw = sh.p[w][0];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float s[2] = {S[0][i], S[1][i]};
      const float mn = fmaxf(m[i], tmax[i]);
      const float corr = m[i] == -INFINITY ? 1.0f : __expf(m[i] - mn);
      const int r = (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      float psum = 0.0f, p[2];
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        p[kt] = s[kt] == -INFINITY ? 0.0f : __expf(s[kt] - mn);
        psum += p[kt];
      }
      uint32_t ph, pl;  // the two keys' (hi, lo) pairs, key tile 0 in the low halves
      split_f16x2(p[0], p[1], ph, pl);
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        const int key = kt * 32 + (lane & 31);
        const int o = r * 64 + (((key >> 3) ^ ((r >> 1) & 7)) << 3) + (key & 7);
        pw[o] = (uint16_t)(ph >> (16 * kt));
        pw[32 * kFK + o] = (uint16_t)(pl >> (16 * kt));
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
      const f16x8 al = *reinterpret_cast<const f16x8 *>(&pw[32 * kFK + oa]);
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

  // normalise and write the rows in the GEMM's split form (one head = one 64-group)
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int t = q0 + w * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
    const float inv = 1.0f / half32_sum(l[i]);
    const float v0 = O[0][i] * inv, v1 = O[1][i] * inv;
    const float gsum = half32_sum(v0 + v1);
    if (t < T) {
      const size_t row = (size_t)t * d + h * 64 + (lane & 31);
      uint32_t hi, lo;
      split_f16x2(v0, v1, hi, lo);
      out.hi[row] = (uint16_t)hi;
      out.lo[row] = (uint16_t)lo;
      out.hi[row + 32] = (uint16_t)(hi >> 16);
      out.lo[row + 32] = (uint16_t)(lo >> 16);
      if ((lane & 31) == 0) out.gs[(size_t)t * (d / 64) + h] = gsum;
    }
  }
}

}  // namespace

size_t attn_kv_split_halves(int n_head, int keys) { return (size_t)n_head * ((keys + kFK - 1) / kFK) * kFK * 64 * 4; }

hipError_t launch_attn_flash(const float *q, int T, int base, const int *kstart, const void *kc, const void *vc,
                             int ld, int n_head, const SplitOut &out, int kvt, hipStream_t s, uint16_t *kv_split,
                             const int *tile_order) {
  if (T <= 0 || base + T > ld) return hipErrorInvalidValue;
  dim3 grid(n_head, (T + kFQ - 1) / kFQ);
  const int d = n_head * 64;
  if (kv_split) {
    // keys 0 .. base + T - 1, padded to whole tiles
    const int L = base + T, Lp = ((L + kFK - 1) / kFK) * kFK;
    const long nthreads = (long)n_head * Lp * 8 + (long)n_head * (Lp / 8) * 64;
    const dim3 sg((unsigned)((nthreads + 255) / 256));
    if (kvt == kKvBf16) {
      hipLaunchKernelGGL(kv_split_kernel<kKvBf16>, sg, dim3(256), 0, s, kc, vc, ld, n_head, L, Lp, kv_split);
      hipLaunchKernelGGL((attn_flash_kernel<kKvBf16, true>), grid, dim3(128), 0, s, q, d, kc, vc, ld, base, T, kstart,
                         out, kv_split, Lp, tile_order);
    } else {
      hipLaunchKernelGGL(kv_split_kernel<kKvF32>, sg, dim3(256), 0, s, kc, vc, ld, n_head, L, Lp, kv_split);
      hipLaunchKernelGGL((attn_flash_kernel<kKvF32, true>), grid, dim3(128), 0, s, q, d, kc, vc, ld, base, T, kstart,
                         out, kv_split, Lp, tile_order);
    }
    return hipGetLastError();
  }
  if (kvt == kKvBf16) {
    hipLaunchKernelGGL((attn_flash_kernel<kKvBf16, false>), grid, dim3(128), 0, s, q, d, kc, vc, ld, base, T, kstart,
                       out, nullptr, 0, tile_order);
  } else {
    hipLaunchKernelGGL((attn_flash_kernel<kKvF32, false>), grid, dim3(128), 0, s, q, d, kc, vc, ld, base, T, kstart,
                       out, nullptr, 0, tile_order);
  }
  return hipGetLastError();
}

}  // namespace itts
