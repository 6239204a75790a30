// Prefill GEMM for gfx950, the activation splitter and the standalone dequantiser.
//
// The GEMM contracts M activation rows against the int8 (or int4) codes on the MFMA
// units (v_mfma_f32_32x32x16_f16).  Codes are exact in fp16, so the matrix cores see the
// true integer weights; activations arrive pre-split as an fp16 pair x = hi + lo (~22
// significant bits) together with their per-64-group row sums, and both halves are
// accumulated in fp32.  The MLX group affine is applied per K group on the fp32 partial:
//   acc += s[n,g] * (sum_{k in g} x[m,k] q[n,k]) + b[n,g] * (sum_{k in g} x[m,k]).
// 4-bit codes enter as the fp16 values 16 + q (bit pattern 0x4C00 | q << 6), so the group
// term uses b - 16 s in place of b.
//
// Block: 512 threads, 2 x 2 worker waves of (32 TM) x (32 TN) outputs, tile (64 TM) x
// (64 TN), and four copier waves.  The K loop runs over 64-wide groups through an NS-stage
// ring of LDS buffers filled by global->LDS DMA (no registers) that only the copiers issue,
// so the copies overlap the workers' MFMAs; each stage holds the hi/lo activation tile, the
// code tile, the group sums and the (scale, bias) pairs.  Activation and code rows are XOR
// swizzled in 16-byte chunks so that the MFMA fragment reads spread over the banks.
// Small M is spread over the chip by splitting K: each split stores its partial tile,
// and the last split to arrive at a tile (wrapping counter) adds the partials in split
// order, so the result does not depend on arrival order.
#include <type_traits>

#include "kernels.h"

namespace itts {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

template <int BITS, int PT, int TM, int TN>
struct Shape {
  static constexpr int BM = 64 * TM, BN = 64 * TN;
  static constexpr int RB = BITS * 8;                          // code bytes per row per group
  static constexpr int A_BYTES = BM * 128;                     // one fp16 plane: 64 values a row
  static constexpr int B_BYTES = BN * RB;
  static constexpr int P_BYTES = BN * (PT == kParamF32 ? 8 : 4);
  static constexpr int OFF_LO = A_BYTES, OFF_B = 2 * A_BYTES, OFF_G = OFF_B + B_BYTES;
  static constexpr int OFF_P = OFF_G + BM * 4, OFF_D = OFF_P + P_BYTES;
  static constexpr int STAGE = OFF_D + 256;                    // + one copy target for padding jobs
  // DMA jobs per stage: 16-byte-per-lane copies of 1 KiB (A planes, codes) and
  // 4-byte-per-lane copies of 256 B (group sums, params), dealt round-robin to the waves
  static constexpr int nA = BM / 4, nB = B_BYTES / 1024, nG = BM / 64, nP = P_BYTES / 256;
  static constexpr int JOBS = nA + nB + nG + nP, PW = (JOBS + 3) / 4;
  static_assert(B_BYTES % 1024 == 0 && P_BYTES % 256 == 0, "tile shape");
};

// LDS on gfx950 has 64 four-byte banks (256 bytes a cycle).  A row of the activation tile
// is 128 bytes, so rows r and r + 1 share one 256-byte bank row; 16-byte chunks are XOR
// swizzled by (r >> 1) & 7 so that the 16 rows a wave reads per cycle hit distinct banks.
// A code row is 64 (8-bit) or 32 (4-bit) bytes; its 16-byte chunks are swizzled by the row's
// position among the rows sharing a bank row.
__device__ __forceinline__ int swz_act(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swz_codes(int bits, int r) { return bits == 8 ? (r >> 2) & 3 : (r >> 3) & 1; }

// Sum over the TPI consecutive lanes of an item: nothing (1) or a DPP quad (4).
template <int TPI>
__device__ __forceinline__ float item_sum(float v) {
  static_assert(TPI == 1 || TPI == 4, "item width");
  if constexpr (TPI == 4) {
    v += dpp_pair<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_pair<0x4E>(v);  // quad_perm [2,3,0,1]
  }
  return v;
}

// two consecutive 8-bit codes (bits sh..sh+15 of w) -> packed fp16 pair (exact)
__device__ __forceinline__ uint32_t f16_pair_u8(uint32_t w, int sh) {
  const float lo = (float)((w >> sh) & 0xffu);
  const float hi = (float)((w >> (sh + 8)) & 0xffu);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// the two nibbles of byte sh/8 of w -> packed fp16 pair (16 + q_even, 16 + q_odd)
__device__ __forceinline__ uint32_t f16_pair_u4(uint32_t w, int sh) {
  const uint32_t b = (w >> sh) & 0xffu;
  return (((b | (b << 12)) & 0x000f000fu) << 6) | 0x4C004C00u;
}

// Global->LDS copies issued by hand: lane l's bytes land at lds + l * size.  The
// compiler cannot tell which ring buffer a pending copy targets, so the builtin makes it
// wait for every copy in flight before any LDS read; issued here, the copies are counted
// by the kernel's own vmcnt waits instead.
// M0 is reserved to the compiler; these kernels use it for nothing else (the copies set
// it themselves before every copy), so the clobber warning is expected.
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(lds_ptr)(p);
}
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// Loads and stores through the global address space (pointers reaching the kernel through
// argument structs are generic to the compiler, and generic accesses count against the
// LDS counter too).
template <class T>
__device__ __forceinline__ T gload(const T *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}
template <class T>
__device__ __forceinline__ void gstore(T *p, T v) {
  *(__attribute__((address_space(1))) T *)p = v;
}
__device__ __forceinline__ void gstore(uint4 *p, uint4 v) {
  *(__attribute__((address_space(1))) u32x4 *)p = u32x4{v.x, v.y, v.z, v.w};
}
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void gstore(float2 *p, float2 v) {
  *(__attribute__((address_space(1))) f32x2v *)p = f32x2v{v.x, v.y};
}

struct Tile {
  int tn, tm, ks;
};

// PROD: 512 threads, waves 4-7 issue every copy and waves 0-3 only compute, so that the
// copies (bound by the CU's vector-memory path) overlap the MFMA and VALU work instead of
// running in series with it inside each wave.
template <int BITS, int PT, int EPI, int KVT, int TM, int TN, int NS, bool PROD>
__global__ __launch_bounds__(PROD ? 512 : 256, (PROD && TM == 1) ? 4 : 1) void gemm_kernel(GemmArgs a, int mode, int nN, int mt, int S, int gps) {
  using Sh = Shape<BITS, PT, TM, TN>;
  constexpr int BM = Sh::BM, BN = Sh::BN, PW = Sh::PW;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
  // copier: issues the copies; worker: computes (both, without PROD).  Wave-uniform.
  const bool copier = !PROD || wave_all >= 4, worker = !PROD || wave_all < 4;
  // the workers' MFMA and VALU instructions issue ahead of the copiers' (235-row prefill
  // 2.41 against 2.45 ms; the copiers raised instead: 2.46 ms)
  if (PROD && worker) __builtin_amdgcn_s_setprio(3);
  const int wave = wave_all & 3;
  const int wm = wave >> 1, wn = wave & 1;
  const int K = a.ql.K, N = a.ql.N, M = a.M, G = K / kGroup;

  // block -> (N tile, M tile, K split).  mode 1 (few M tiles): blocks that read the same
  // codes sit on one XCD (dispatch deals blocks to the 8 XCDs round-robin).
  Tile t;
  {
    const int b = blockIdx.x;
    if (mode == 1) {
      const int y = b >> 3;
      const int w = (y / mt) * 8 + (b & 7);
      if (w >= nN * S) return;
      t.tm = y % mt;
      t.tn = w / S;
      t.ks = w - t.tn * S;
    } else {
      t.tn = b % nN;
      const int r = b / nN;
      t.tm = r % mt;
      t.ks = r / mt;
    }
  }
  const int m0 = t.tm * BM, n0 = t.tn * BN;
  const int g0 = t.ks * gps, ng = min(G, g0 + gps) - g0;

  const uint8_t *codes = a.ql.codes;
  const size_t code_row = (size_t)K * BITS / 8;

  // one stage's copies: exactly PW DMA instructions per wave, so vmcnt counts stages
  auto issue = [&](int g, char *st) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < PW; s++) {
      const int j = s * 4 + wave;
      if (j < Sh::nA) {
        const int plane = j / (BM / 8), c1k = j % (BM / 8);
        const int r = c1k * 8 + (lane >> 3);
        const int lc = (lane & 7) ^ swz_act(r);
        const int m = min(m0 + r, M - 1);
        const uint16_t *src = (plane ? a.x.lo : a.x.hi) + (size_t)m * K + g * kGroup + lc * 8;
        dma16(src, lds_addr(st + plane * Sh::A_BYTES + c1k * 1024));
      } else if (j < Sh::nA + Sh::nB) {
        constexpr int CR = Sh::RB / 16, RPB = 1024 / Sh::RB;
        const int jb = j - Sh::nA;
        const int r = jb * RPB + lane / CR;
        const int lc = (lane % CR) ^ swz_codes(BITS, r);
        const int n = min(n0 + r, N - 1);
        const uint8_t *src = codes + (size_t)n * code_row + g * Sh::RB + lc * 16;
        dma16(src, lds_addr(st + Sh::OFF_B + jb * 1024));
      } else if (j < Sh::nA + Sh::nB + Sh::nG) {
        const int jg = j - Sh::nA - Sh::nB;
        const int m = min(m0 + jg * 64 + lane, M - 1);
        dma4(a.x.gs + (size_t)m * G + g, lds_addr(st + Sh::OFF_G + jg * 256));
      } else if (j < Sh::JOBS) {
        const int jp = j - Sh::nA - Sh::nB - Sh::nG;
        const int e = jp * 64 + lane;
        if constexpr (PT == kParamF32) {
          const int n = min(n0 + (e >> 1), N - 1);
          const float *src = static_cast<const float *>(a.ql.params) + ((size_t)n * G + g) * 2 + (e & 1);
          dma4(src, lds_addr(st + Sh::OFF_P + jp * 256));
        } else {
          const int n = min(n0 + e, N - 1);
          const uint32_t *src = static_cast<const uint32_t *>(a.ql.params) + (size_t)n * G + g;
          dma4(src, lds_addr(st + Sh::OFF_P + jp * 256));
        }
      } else {
        dma4(a.x.gs + g, lds_addr(st + Sh::OFF_D));
      }
    }
  };

  floatx16 acc[TM][TN], P0[TM][TN], P1[TM][TN];
  float2 sbp[TN];
  floatx4 gsp[TM][4];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  auto mma = [&](const char *st, floatx16(&P)[TM][TN]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) P[i][j][e] = 0.0f;
    // K order inside a group: lane half h = lane >> 5 of MFMA step kk = 2 kp + s takes the 8
    // values 32 kp + 16 h + 8 s .. +7 (the same permutation for activations and codes, so
    // the contraction is unchanged); a lane's codes for both steps of a pair are then one
    // contiguous 16-byte (8-bit) or 8-byte (4-bit) read.
#pragma unroll
    for (int kp = 0; kp < 2; kp++) {
      const int h = lane >> 5;
      f16x8 bq[2][TN];
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int nr = wn * 32 * TN + j * 32 + (lane & 31);
        if constexpr (BITS == 8) {
          const u32x4 q =
              *reinterpret_cast<const u32x4 *>(st + Sh::OFF_B + nr * 64 + (((2 * kp + h) ^ swz_codes(8, nr)) << 4));
          const u32x4 b0 = {f16_pair_u8(q[0], 0), f16_pair_u8(q[0], 16), f16_pair_u8(q[1], 0), f16_pair_u8(q[1], 16)};
          const u32x4 b1 = {f16_pair_u8(q[2], 0), f16_pair_u8(q[2], 16), f16_pair_u8(q[3], 0), f16_pair_u8(q[3], 16)};
          bq[0][j] = __builtin_bit_cast(f16x8, b0);
          bq[1][j] = __builtin_bit_cast(f16x8, b1);
        } else {
          const uint2 q =
              *reinterpret_cast<const uint2 *>(st + Sh::OFF_B + nr * 32 + ((kp ^ swz_codes(4, nr)) << 4) + h * 8);
          const u32x4 b0 = {f16_pair_u4(q.x, 0), f16_pair_u4(q.x, 8), f16_pair_u4(q.x, 16), f16_pair_u4(q.x, 24)};
          const u32x4 b1 = {f16_pair_u4(q.y, 0), f16_pair_u4(q.y, 8), f16_pair_u4(q.y, 16), f16_pair_u4(q.y, 24)};
          bq[0][j] = __builtin_bit_cast(f16x8, b0);
          bq[1][j] = __builtin_bit_cast(f16x8, b1);
        }
      }
#pragma unroll
      for (int sub = 0; sub < 2; sub++) {
        f16x8 ah[TM], al[TM];
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const int row = wm * 32 * TM + i * 32 + (lane & 31);
          const int c = 4 * kp + 2 * h + sub;
          const int off = row * 128 + ((c ^ swz_act(row)) << 4);
          ah[i] = *reinterpret_cast<const f16x8 *>(st + off);
          al[i] = *reinterpret_cast<const f16x8 *>(st + Sh::OFF_LO + off);
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++) {
            P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bq[sub][j], P[i][j], 0, 0, 0);
            P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bq[sub][j], P[i][j], 0, 0, 0);
          }
      }
    }
  };

  // (scale, bias) of this wave's columns, for the group in st
  auto read_params = [&](const char *st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int nr = wn * 32 * TN + j * 32 + (lane & 31);
      float2 sb;
      if constexpr (PT == kParamF32) {
        sb = *reinterpret_cast<const float2 *>(st + Sh::OFF_P + nr * 8);
      } else {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(st + Sh::OFF_P + nr * 4);
        sb = make_float2(half_bits_to_float(w & 0xffffu), half_bits_to_float(w >> 16));
      }
      if constexpr (BITS == 4) sb.y = sb.y - 16.0f * sb.x;
      sbp[j] = sb;
    }
  };
  // ... and the group sums of its rows
  auto read_group = [&](const char *st) __attribute__((always_inline)) {
    read_params(st);
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int rb = wm * 32 * TM + i * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int q = 0; q < 4; q++) gsp[i][q] = *reinterpret_cast<const floatx4 *>(st + Sh::OFF_G + (rb + q * 8) * 4);
    }
  };

  auto apply = [&](const floatx16(&P)[TM][TN]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++)
          acc[i][j][e] = fmaf(sbp[j].x, P[i][j][e], fmaf(sbp[j].y, gsp[i][e >> 2][e & 3], acc[i][j][e]));
  };

  // The fold straight from the stage in LDS (128 x 128 tiles): the group sums of one M
  // sub-tile at a time are held in registers, so the fold adds 16 registers to the
  // partial tile instead of 32 (those tiles run at the 256-register limit).
  auto apply_from = [&](const char *st, const floatx16(&P)[TM][TN]) __attribute__((always_inline)) {
    read_params(st);
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int rb = wm * 32 * TM + i * 32 + (lane >> 5) * 4;
      floatx4 g[4];
#pragma unroll
      for (int q = 0; q < 4; q++) g[q] = *reinterpret_cast<const floatx4 *>(st + Sh::OFF_G + (rb + q * 8) * 4);
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++)
          acc[i][j][e] = fmaf(sbp[j].x, P[i][j][e], fmaf(sbp[j].y, g[e >> 2][e & 3], acc[i][j][e]));
    }
  };

  auto stage = [&](int i) __attribute__((always_inline)) { return lds + (i % NS) * Sh::STAGE; };

  // group i: wait for its copies, start the copies NS-1 groups ahead into the buffer that
  // group i-1 used, contract, then fold group i-1's partial (its params were read into
  // registers while the buffer was still valid)
  auto step = [&](int i, floatx16(&Pc)[TM][TN], const floatx16(&Pp)[TM][TN]) __attribute__((always_inline)) {
    if (copier) {
      const int ahead = min(NS - 2, ng - 1 - i);
      if (ahead <= 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      } else if (ahead == 1) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PW) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PW) : "memory");
      }
    }
    __syncthreads();
    if (copier && i + NS - 1 < ng) issue(g0 + i + NS - 1, stage(i + NS - 1));
    if (worker) {
      if constexpr (PROD) {
        // 128 x 128 tiles at two waves per SIMD: the group's affine is applied at once, so
        // only one partial tile is live (the other wave on the SIMD covers the MFMA latency)
        mma(stage(i), Pc);
        apply_from(stage(i), Pc);
      } else {
        mma(stage(i), Pc);
        if (i > 0) apply(Pp);
        read_group(stage(i));
      }
    }
  };

  if (copier)
    for (int i = 0; i < NS - 1 && i < ng; i++) issue(g0 + i, stage(i));
  // Folded LayerNorm input: each row's mean and rstd from its groups' statistics.  A quad of
  // worker lanes a row (64 rows per pass of the four worker waves), lane p of the quad
  // holding groups p, p + 4, ... (K <= 2048: at most 8), the quad's sums formed by two DPP
  // quad permutes.  On 64-row tiles the loads are issued here, before the K loop (nothing
  // else of the workers' waits on the vector-memory counter), and reduced after it; 128-row
  // tiles (no registers to spare) load after the loop.
  constexpr bool kFoldIn = EPI == kEpiQKV || EPI == kEpiGelu;
  constexpr int kFoldGpl = 8;  // groups a lane
  constexpr bool kFoldEarly = kFoldIn && TM == 1;
  __shared__ float2 fold_row[kFoldIn ? BM : 1];
  const bool fin = kFoldIn && a.tfi.st != nullptr;
  float2 fv[kFoldEarly ? kFoldGpl : 1];
  auto fold_load = [&](int pass, float2 *v) __attribute__((always_inline)) {
    const int m = min(m0 + pass * 64 + ((tid & 255) >> 2), M - 1), p = tid & 3;
#pragma unroll
    for (int i = 0; i < kFoldGpl; i++) {
      const int g = p + 4 * i;
      v[i] = g < G ? a.tfi.st[(size_t)m * G + g] : make_float2(0.0f, 0.0f);
    }
  };
  auto fold_reduce = [&](int pass, const float2 *v) __attribute__((always_inline)) {
    const int p = tid & 3;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kFoldGpl; i++) sum += v[i].x;
    sum += dpp_pair<0xB1>(sum);  // quad_perm [1,0,3,2]
    sum += dpp_pair<0x4E>(sum);  // quad_perm [2,3,0,1]
    const float mean = sum / (float)G;
    float m2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kFoldGpl; i++) {
      const float dm = v[i].x - mean;
      if (p + 4 * i < G) m2 += v[i].y + 64.0f * (dm * dm);
    }
    m2 += dpp_pair<0xB1>(m2);
    m2 += dpp_pair<0x4E>(m2);
    if (p == 0) fold_row[pass * 64 + ((tid & 255) >> 2)] = make_float2(mean, 1.0f / sqrtf(m2 / (float)K + 1e-5f));
  };
  if constexpr (kFoldEarly) {
    if (fin && worker) fold_load(0, fv);
  }
  // The epilogue's column constants on 64 x 64 tiles (one 32-column MFMA tile a wave): the
  // bias (or the folded LayerNorm's c) and the folded G of the lane's column, loaded here so
  // the epilogue does not start with a memory round trip.  Addresses selected, not loads
  // predicated (a load behind a branch would make the compiler wait for the fold loads).
  constexpr bool kColEarly = PROD && TM == 1 && TN == 1;
  float cb = 0.0f, cg = 0.0f;
  if constexpr (kColEarly) {
    if (worker) {
      const int n = min(n0 + wn * 32 + (lane & 31), N - 1);
      cb = gload((kFoldIn && fin ? a.tfi.c : a.ql.bias) + n);
      if constexpr (kFoldIn) cg = gload((fin ? a.tfi.G : a.ql.bias) + n);
    }
  }
  // ... and the residual fold-out's gamma: worker thread t takes columns 16 (t & 3) .. +15
  // of the tile (its item in the epilogue below), the same for every row
  constexpr bool kGamEarly = kColEarly && EPI == kEpiResid;
  float gam0[kGamEarly ? 16 : 1];
  if constexpr (kGamEarly) {
    if (worker && a.tfo.st) {
      const float *gp = a.tfo.gamma + n0 + (tid & 3) * 16;
#pragma unroll
      for (int c = 0; c < 16; c++) gam0[c] = gload(gp + c);
    }
  }
  int i = 0;
  for (; i + 1 < ng; i += 2) {
    step(i, P0, P1);
    step(i + 1, P1, P0);
  }
  if (i < ng) {
    step(i, P0, P1);
    if (worker && !PROD) apply(P0);
  } else {
    if (worker && !PROD) apply(P1);
  }

  if constexpr (kFoldIn) {
    if (fin && worker) {
      if constexpr (kFoldEarly) {
        fold_reduce(0, fv);
      } else {
#pragma unroll
        for (int pass = 0; pass < TM; pass++) {
          float2 v[kFoldGpl];
          fold_load(pass, v);
          fold_reduce(pass, v);
        }
      }
    }
    if (fin) __syncthreads();  // rows reduced by one wave are read by the others
  }

  // Residual epilogues on 64-row tiles: the lane's old rows y, all loaded before any is
  // used.  Read and written element by element, each load waited behind the previous
  // element's store (the compiler cannot move a load of y above a store to y): 16 round
  // trips a lane.
  constexpr bool kResid = EPI == kEpiResid;
  float yv[kResid ? TM : 1][kResid ? TN : 1][kResid ? 16 : 1];
  auto load_y = [&]() __attribute__((always_inline)) {
    if constexpr (kResid) {
#pragma unroll
      for (int i2 = 0; i2 < TM; i2++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          // indexes clamped rather than loads predicated: one straight run of loads, which
          // the compiler's wait counting follows exactly (behind branches it waits for every
          // access in flight, the stores of earlier elements included)
          const int n = min(n0 + wn * 32 * TN + j * 32 + (lane & 31), N - 1);
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const int m = min(m0 + wm * 32 * TM + i2 * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3), M - 1);
            yv[i2][j][e] = gload<float>(a.y + (size_t)m * N + n);
          }
        }
    }
  };

  const int tile = t.tm * nN + t.tn;
  if (S > 1) {
    // Partial tiles in the MFMA register order (8 bytes per access, contiguous across the
    // wave).  They travel through agent-scope (sc1) stores and loads, which are coherent
    // across the XCDs' L2s, so no L2 write-back fence is needed: each thread's stores are
    // complete (vmcnt 0) before the block's arrival is counted, and the last block's loads
    // are issued after it has seen the count.
    constexpr int TILE = BM * BN;
    uint64_t *wsb = reinterpret_cast<uint64_t *>(a.ws + (size_t)tile * S * TILE);
    uint64_t *mine = wsb + (size_t)t.ks * (TILE / 2);
    // register pair h of sub-tile i2 holds rows from `dead` on only when every one of its
    // rows is past M (few-row tiles): those pairs are neither stored nor summed
    auto dead = [&](int i2, int h) {
      return m0 + wm * 32 * TM + i2 * 32 + (h >> 1) * 8 + ((2 * h) & 3) >= M;
    };
    if (worker) {
#pragma unroll
      for (int i2 = 0; i2 < TM; i2++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int h = 0; h < 8; h++) {
            if (dead(i2, h)) continue;
            const float2 v = make_float2(acc[i2][j][2 * h], acc[i2][j][2 * h + 1]);
            __hip_atomic_store(mine + ((((wave * TM + i2) * TN + j) * 8 + h) * 64 + lane),
                               __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) last_flag = atomicInc(a.cnt + tile, (uint32_t)(S - 1)) == (uint32_t)(S - 1) ? 1u : 0u;
    __syncthreads();
    if (!last_flag) return;
    // (the old rows' loads go out ahead of the partials', their latencies overlapping; on
    // 128-row tiles, whose registers are full here, after them)
    if (kResid && TM == 1 && worker) load_y();
    // splits added in split order (the block's own partial from registers)
    if (worker) {
#pragma unroll
      for (int i2 = 0; i2 < TM; i2++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          const size_t base = (size_t)(((wave * TM + i2) * TN + j) * 8) * 64 + lane;
          floatx16 sum;
          for (int s2 = 0; s2 < S; s2++) {
            floatx16 v;
            if (s2 == t.ks) {
              v = acc[i2][j];
            } else {
#pragma unroll
              for (int h = 0; h < 8; h++) {
                if (dead(i2, h)) {
                  v[2 * h] = 0.0f;
                  v[2 * h + 1] = 0.0f;
                  continue;
                }
                const float2 w = __builtin_bit_cast(
                    float2, __hip_atomic_load(wsb + (size_t)s2 * (TILE / 2) + base + h * 64, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT));
                v[2 * h] = w.x;
                v[2 * h + 1] = w.y;
              }
            }
            sum = s2 == 0 ? v : sum + v;
          }
          acc[i2][j] = sum;
        }
    }
  }

  if (kResid && S == 1 && TM == 1 && worker) load_y();

  if constexpr (EPI == kEpiResid) {
    if (a.tfo.st) {
      // The updated rows x staged in LDS, then per (row, 64-column group): the group's mean
      // and sum of squared deviations of x, and gamma * x as the next GEMM's input (hi/lo
      // planes and the group sum).
      constexpr int LDT = BN + 1;
      constexpr int GPR = BN / 64, ITEMS = BM * GPR, TPI = 256 / ITEMS, VPT = 64 / TPI;
      static_assert(ITEMS * TPI == 256 && VPT % 8 == 0, "fold epilogue shape");
      float *T = reinterpret_cast<float *>(lds);
      // this thread's item (row rl, 64-column group grp, values c0 .. c0 + VPT - 1); its
      // gamma values (16-byte aligned: the vector starts on 256 bytes and c0 is a multiple
      // of 16) are loaded under the staging below on 64-row tiles, after it on 128-row
      // tiles (whose registers the staged tile still holds)
      const int item = tid / TPI, sub = tid % TPI;
      const int rl = item / GPR, grp = item % GPR;
      const int c0 = grp * 64 + sub * VPT;
      // N is a multiple of 64: a group is wholly in or out
      const bool live = worker && m0 + rl < M && n0 + c0 < N;
      float4 gam[VPT / 4];
      auto load_gamma = [&]() __attribute__((always_inline)) {
        if constexpr (kGamEarly) {
          static_assert(VPT == 16 && TPI == 4, "gamma loaded before the K loop for 16-column items");
#pragma unroll
          for (int c = 0; c < 4; c++) gam[c] = make_float4(gam0[4 * c], gam0[4 * c + 1], gam0[4 * c + 2], gam0[4 * c + 3]);
        } else {
#pragma unroll
          for (int c = 0; c < VPT / 4; c++)
            gam[c] = live ? reinterpret_cast<const float4 *>(a.tfo.gamma + n0 + c0)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      };
      if constexpr (TM == 1) load_gamma();
      __syncthreads();
      if (worker)
#pragma unroll
        for (int i2 = 0; i2 < TM; i2++)
#pragma unroll
          for (int j = 0; j < TN; j++) {
            const int cl = wn * 32 * TN + j * 32 + (lane & 31), n = n0 + cl;
            if (n >= N) continue;
            const float bias = kColEarly ? cb : a.ql.bias[n];
            const int rb = wm * 32 * TM + i2 * 32 + (lane >> 5) * 4;  // tile row of element 0
            // values first (straight-line), then the stores predicated on the row
            float outv[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
              const float y = TM == 1 ? yv[i2][j][e]
                                      : gload(a.y + (size_t)min(m0 + rb + (e >> 2) * 8 + (e & 3), M - 1) * N + n);
              outv[e] = y + (acc[i2][j][e] + bias);
              T[(rb + (e >> 2) * 8 + (e & 3)) * LDT + cl] = outv[e];
            }
#pragma unroll
            for (int e = 0; e < 16; e++) asm volatile("" : "+v"(outv[e]));
#pragma unroll
            for (int e = 0; e < 16; e++) {
              const int m = m0 + rb + (e >> 2) * 8 + (e & 3);
              if (m < M) gstore(a.y + (size_t)m * N + n, outv[e]);
            }
          }
      __syncthreads();
      if constexpr (TM != 1) load_gamma();
      if (worker) {
        const int m = m0 + rl, n = n0 + c0;
        float xv[VPT];
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < VPT; c++) {
          xv[c] = T[rl * LDT + c0 + c];
          sum += xv[c];
        }
        sum = item_sum<TPI>(sum);
        const float mean = sum / 64.0f;
        float m2 = 0.0f, gsum = 0.0f;
#pragma unroll
        for (int c = 0; c < VPT; c += 8) {
          uint32_t hw[4], lw[4];
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const float v0 = xv[c + e], v1 = xv[c + e + 1];
            const float d0 = v0 - mean, d1 = v1 - mean;
            m2 += d0 * d0;
            m2 += d1 * d1;
            const float4 gq = gam[(c + e) >> 2];
            const float g0 = ((e & 2) ? gq.z : gq.x) * v0;
            const float g1 = ((e & 2) ? gq.w : gq.y) * v1;
            gsum += g0;
            gsum += g1;
            split_f16x2(g0, g1, hw[e >> 1], lw[e >> 1]);
          }
          if (live) {
            gstore(reinterpret_cast<uint4 *>(a.tfo.o.hi + (size_t)m * N + n + c), make_uint4(hw[0], hw[1], hw[2], hw[3]));
            gstore(reinterpret_cast<uint4 *>(a.tfo.o.lo + (size_t)m * N + n + c), make_uint4(lw[0], lw[1], lw[2], lw[3]));
          }
        }
        m2 = item_sum<TPI>(m2);
        gsum = item_sum<TPI>(gsum);
        if (live && sub == 0) {
          const size_t gi = (size_t)m * (N / kGroup) + (n0 + grp * 64) / kGroup;
          gstore(a.tfo.o.gs + gi, gsum);
          gstore(a.tfo.st + gi, make_float2(mean, m2));
        }
      }
      return;
    }
  }

  if constexpr (EPI == kEpiGelu) {
    // GELU tile staged in LDS, then written as the next GEMM's input: hi/lo planes and
    // the per-64-column row sums
    constexpr int LDT = BN + 1;
    float *T = reinterpret_cast<float *>(lds);
    __syncthreads();
    if (worker)
#pragma unroll
    for (int i2 = 0; i2 < TM; i2++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int cl = wn * 32 * TN + j * 32 + (lane & 31);
        const bool nl = n0 + cl < N;
        const float bias = kColEarly ? cb : nl ? (fin ? a.tfi.c[n0 + cl] : a.ql.bias[n0 + cl]) : 0.0f;
        const float gn = kColEarly ? (fin ? cg : 0.0f) : fin && nl ? a.tfi.G[n0 + cl] : 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int rl = wm * 32 * TM + i2 * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          float v = acc[i2][j][e];
          if (fin) v = fold_row[rl].y * (v - fold_row[rl].x * gn);
          T[rl * LDT + cl] = gelu_tanh_exp(v + bias);
        }
      }
    __syncthreads();
    constexpr int GPR = BN / 64, ITEMS = BM * GPR, TPI = 256 / ITEMS, VPT = 64 / TPI;
    static_assert(ITEMS * TPI == 256 && VPT % 8 == 0, "gelu epilogue shape");
    if (worker) {
      const int item = tid / TPI, sub = tid % TPI;
      const int rl = item / GPR, grp = item % GPR;
      const int c0 = grp * 64 + sub * VPT;
      const int m = m0 + rl, n = n0 + c0;
      float sum = 0.0f;
      const bool live = m < M && n < N;
#pragma unroll
      for (int c = 0; c < VPT; c += 8) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float v0 = T[rl * LDT + c0 + c + e], v1 = T[rl * LDT + c0 + c + e + 1];
          sum += v0;
          sum += v1;
          split_f16x2(v0, v1, hw[e >> 1], lw[e >> 1]);
        }
        if (live) {
          gstore(reinterpret_cast<uint4 *>(a.xo.hi + (size_t)m * N + n + c), make_uint4(hw[0], hw[1], hw[2], hw[3]));
          gstore(reinterpret_cast<uint4 *>(a.xo.lo + (size_t)m * N + n + c), make_uint4(lw[0], lw[1], lw[2], lw[3]));
        }
      }
      sum = item_sum<TPI>(sum);
      if (live && sub == 0) gstore(a.xo.gs + (size_t)m * (N / kGroup) + n / kGroup, sum);
    }
    return;
  } else if (worker) {
#pragma unroll
    for (int i2 = 0; i2 < TM; i2++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * 32 * TN + j * 32 + (lane & 31);
        if (n >= N) continue;
        const float bias = kColEarly ? cb : fin ? a.tfi.c[n] : a.ql.bias[n];
        const float gn = kColEarly ? (fin ? cg : 0.0f) : fin ? a.tfi.G[n] : 0.0f;
        const int rb = wm * 32 * TM + i2 * 32 + (lane >> 5) * 4;  // tile row of element 0
        // 128-row tiles: the sub-tile's 16 old values loaded together (registers for all 64
        // of the lane's would spill)
        float ysub[kResid && TM != 1 ? 16 : 1];
        if constexpr (kResid && TM != 1) {
#pragma unroll
          for (int e = 0; e < 16; e++)
            ysub[e] = gload(a.y + (size_t)min(m0 + rb + (e >> 2) * 8 + (e & 3), M - 1) * N + n);
        }
        // The sub-tile's values first, in straight-line code (the waits on its loads come
        // here, once), then the stores, each predicated on its row: behind a predicate the
        // compiler's wait counting waits for every access in flight, earlier stores too.
        float outv[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int rl = rb + (e >> 2) * 8 + (e & 3);
          float v = acc[i2][j][e];
          if constexpr (kFoldIn) v = fin ? fold_row[rl].y * (v - fold_row[rl].x * gn) : v;
          v += bias;
          if constexpr (kResid) v = (TM == 1 ? yv[i2][j][e] : ysub[e]) + v;
          outv[e] = v;
        }
        // (an empty asm over the values keeps the compiler from sinking their arithmetic,
        // and the waits on its operands, into the predicated stores)
#pragma unroll
        for (int e = 0; e < 16; e++) asm volatile("" : "+v"(outv[e]));
        // stores through the global address space (generic stores also count against the
        // LDS counter)
        if constexpr (EPI == kEpiStore || EPI == kEpiResid) {
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const int m = m0 + rb + (e >> 2) * 8 + (e & 3);
            if (m < M) gstore(a.y + (size_t)m * N + n, outv[e]);
          }
        } else {
          const int d = a.qkv.d_model;
          if (n < d) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
              const int m = m0 + rb + (e >> 2) * 8 + (e & 3);
              if (m < M) gstore(a.qkv.q_out + (size_t)m * d + n, outv[e]);
            }
          } else {
            const bool is_k = n < 2 * d;
            const int idx = is_k ? n - d : n - 2 * d;
            const int h = idx >> 6, e2 = idx & 63;
            auto put = [&](void *cache, int pos, float v) __attribute__((always_inline)) {
              const size_t ci = ((size_t)h * a.qkv.max_seq + pos) * kHeadDim + e2;
              if constexpr (KVT == kKvBf16) {
                gstore(static_cast<uint16_t *>(cache) + ci, (uint16_t)float_to_bf16_bits(v));
              } else {
                gstore(static_cast<float *>(cache) + ci, v);
              }
            };
            if (!a.qkv.seqs) {
              void *cache = is_k ? a.qkv.k_cache : a.qkv.v_cache;
#pragma unroll
              for (int e = 0; e < 16; e++) {
                const int m = m0 + rb + (e >> 2) * 8 + (e & 3);
                if (m < M) put(cache, a.qkv.pos0 + m, outv[e]);
              }
            } else {  // batched decode: row m is sequence m
#pragma unroll
              for (int e = 0; e < 16; e++) {
                const int m = m0 + rb + (e >> 2) * 8 + (e & 3);
                if (m >= M) continue;
                const BatchSeq *sq = a.qkv.seqs + m;
                DecodeCtl *ctl = gload(&sq->ctl);
                if (gload<int32_t>(&ctl->done)) continue;
                put(static_cast<char *>(gload(is_k ? &sq->k : &sq->v)) + a.qkv.layer_off * (KVT == kKvBf16 ? 2 : 4),
                    gload<int32_t>(&ctl->valid_len), outv[e]);
              }
            }
          }
        }
      }
  }
}

// ---- few-row products (M <= 8: the batched decode step) ---------------------------------
// The 64-row tiles above spend most of a launch filling the ring for a few real rows.  Here
// a block of kFewWaves waves takes 64 output columns (two 32-column MFMA tiles) over
// kFewWaves K groups, one per wave, with no LDS staging: each lane loads its activation and code
// fragments straight into registers (a lane's 16 codes of a column are one 16-byte load,
// its 16 activations of a row two), in the K order the tiles above use.  Rows past M are
// zero fragments; in the 32 x 32 result a lane's rows 4h .. 4h+3 (h = lane >> 5) are the
// only live ones.  The waves' partials are added in wave order in LDS; the K splits
// (blocks) in split order by the last block of the column tile to arrive, as above.
// One K group per wave (K <= 8192; longer K takes the tiled GEMM): the register arrays
// sized for one group keep the kernel at 92-98 VGPRs (128-132 with the folded LayerNorm),
// so two blocks share a compute unit and mel_head's 387 blocks run in one round (batched
// decode 5,915 -> 6,134 tok/s against arrays sized for two groups).
constexpr int kFewRows = 8, kFewMaxGw = 1, kFewMaxSplits = 16;
// eight waves per block measured 3 % faster on batched decode than four (half the K
// splits) and 23 % faster than two
constexpr int kFewWaves = 8;                  // waves per block, a K group each
constexpr int kFewEPT = 512 / (64 * kFewWaves);  // of a tile's 8 x 64 results, per thread

// With FOLD (a.fold, one group a wave), row c's activations are gamma * x read from the fp32
// rows and split to hi/lo here, their group sums formed here, and wave w forms the mean and
// rstd of row w (biased variance, eps 1e-5, over K/256 float4s a lane in registers) beside
// the product; the epilogue takes rstd (sum - mean G[n]) + c[n].
constexpr int kFoldQ = 8;  // float4s a lane of a row's statistics: K <= 2048
template <int BITS, int PT, int EPI, int KVT, bool FOLD>
__global__ __launch_bounds__(64 * kFewWaves) void few_kernel(GemmArgs a, int nN, int S, int gw) {
  __shared__ float red[kFewWaves][512];
  __shared__ float gel[kFewRows][65];
  __shared__ float row_mu[kFewRows], row_rs[kFewRows];
  __shared__ uint32_t last_flag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, c = lane & 31;
  const int tn = blockIdx.x % nN, ks = blockIdx.x / nN;
  const int N = a.ql.N, K = a.ql.K, G = K / kGroup, M = a.M;
  const int n0 = tn * 64;
  // the epilogue's operands of this thread's results (entry i = tid + 512 q -> row
  // m = 4 (i & 63) / 32 + (i >> 6) % 4, column n0 + 32 (i >> 8) + i % 32), loaded first so
  // that their latency passes during the product; only the tile's last block uses them
  float ep_b[kFewEPT], ep_g[kFewEPT], ep_y[kFewEPT];
  BatchSeq ep_sq[kFewEPT];
#pragma unroll
  for (int q = 0; q < kFewEPT; q++) {
    const int i = tid + 64 * kFewWaves * q, ln = i & 63;
    const int m = 4 * (ln >> 5) + ((i >> 6) & 3), n = min(n0 + 32 * (i >> 8) + (ln & 31), N - 1);
    ep_b[q] = FOLD ? a.fold.c[n] : a.ql.bias[n];
    ep_g[q] = FOLD ? a.fold.G[n] : 0.0f;
    ep_y[q] = EPI == kEpiResid && m < M ? a.y[(size_t)m * N + n] : 0.0f;
    if constexpr (EPI == kEpiQKV)
      if (a.qkv.seqs) ep_sq[q] = a.qkv.seqs[min(m, M - 1)];
  }
  // this wave's groups: ks * 4 gw + 4 i + wave, i < gw (none past G)
  floatx4 acc[2] = {floatx4{0.0f, 0.0f, 0.0f, 0.0f}, floatx4{0.0f, 0.0f, 0.0f, 0.0f}};
  u32x4 xa[kFewMaxGw][2][2][2];  // [group][plane][kp][half]: row c, K 32 kp + 16 h .. +15
  u32x4 cq[kFewMaxGw][2][2];     // [group][j][kp] (8-bit: 16 codes; 4-bit: 16 nibbles in .x, .y)
  // parameters stay raw until the products (converting them here would wait for each
  // group's loads in turn)
  using PRaw = typename std::conditional<PT == kParamF16, uint32_t, float2>::type;
  PRaw pr[kFewMaxGw][2];
  float gsr[kFewMaxGw][4];       // group sums of the lane's live rows 4h + e
  float4 xf[2][4];               // FOLD: row c, K 64 g + 32 kp + 16 h + 4 q .. +3 (gamma * x)
  float4 st[kFoldQ];             // FOLD: row `wave`, float4s lane + 64 i
#pragma unroll
  for (int gi = 0; gi < kFewMaxGw; gi++) {
    const int g = ks * kFewWaves * gw + kFewWaves * gi + wave;
    const bool live = gi < gw && g < G;
#pragma unroll
    for (int p2 = 0; p2 < 2; p2++)
#pragma unroll
      for (int kp = 0; kp < 2; kp++)
#pragma unroll
        for (int q = 0; q < 2; q++) xa[gi][p2][kp][q] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (FOLD) {
      if (gi == 0) {
#pragma unroll
        for (int kp = 0; kp < 2; kp++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int k = g * kGroup + 32 * kp + 16 * h + 4 * q;
            xf[kp][q] = live && c < M ? reinterpret_cast<const float4 *>(a.fold.x + (size_t)c * K)[k >> 2]
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          }
      }
    } else if (live && c < M) {
      const size_t off = (size_t)c * K + (size_t)g * kGroup + 16 * h;
#pragma unroll
      for (int kp = 0; kp < 2; kp++) {
        const u32x4 *ph = reinterpret_cast<const u32x4 *>(a.x.hi + off + 32 * kp);
        const u32x4 *pl = reinterpret_cast<const u32x4 *>(a.x.lo + off + 32 * kp);
        xa[gi][0][kp][0] = ph[0];
        xa[gi][0][kp][1] = ph[1];
        xa[gi][1][kp][0] = pl[0];
        xa[gi][1][kp][1] = pl[1];
      }
    }
    // code fragments of columns n0 + 32 j + c (a column past N reads column N - 1, a group
    // past G reads group 0)
    const int gl = live ? g : 0;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = min(n0 + 32 * j + c, N - 1);
#pragma unroll
      for (int kp = 0; kp < 2; kp++) {
        if constexpr (BITS == 8) {
          cq[gi][j][kp] =
              *reinterpret_cast<const u32x4 *>(a.ql.codes + (size_t)n * K + (size_t)gl * 64 + 32 * kp + 16 * h);
        } else {
          const uint2 v =
              *reinterpret_cast<const uint2 *>(a.ql.codes + (size_t)n * (K / 2) + (size_t)gl * 32 + 16 * kp + 8 * h);
          cq[gi][j][kp] = u32x4{v.x, v.y, 0u, 0u};
        }
      }
      pr[gi][j] = static_cast<const PRaw *>(a.ql.params)[(size_t)n * G + gl];
    }
    if constexpr (!FOLD) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int m = 4 * h + e;
        gsr[gi][e] = live && m < M ? a.x.gs[(size_t)m * G + g] : 0.0f;
      }
    }
  }
  if constexpr (FOLD) {
    // gamma * x as hi/lo fp16 and the lane's share of row c's group sum (the other 32
    // values are in lane c ^ 32)
    const int g = ks * kFewWaves * gw + wave;
    if (g < G) {
      float gsum = 0.0f;
#pragma unroll
      for (int kp = 0; kp < 2; kp++)
#pragma unroll
        for (int sub = 0; sub < 2; sub++) {
          uint32_t hw[4], lw[4];
#pragma unroll
          for (int q2 = 0; q2 < 2; q2++) {
            const int k = g * kGroup + 32 * kp + 16 * h + 8 * sub + 4 * q2;
            const float4 gm = reinterpret_cast<const float4 *>(a.fold.gamma)[k >> 2];
            const float4 v = xf[kp][2 * sub + q2];
            const float y[4] = {v.x * gm.x, v.y * gm.y, v.z * gm.z, v.w * gm.w};
#pragma unroll
            for (int e2 = 0; e2 < 2; e2++) {
              gsum += y[2 * e2] + y[2 * e2 + 1];
              split_f16x2(y[2 * e2], y[2 * e2 + 1], hw[2 * q2 + e2], lw[2 * q2 + e2]);
            }
          }
          xa[0][0][kp][sub] = u32x4{hw[0], hw[1], hw[2], hw[3]};
          xa[0][1][kp][sub] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        }
      gsum += __shfl_xor(gsum, 32, 64);
#pragma unroll
      for (int e = 0; e < 4; e++) gsr[0][e] = __shfl(gsum, 4 * h + e, 64);
    }
    // this wave's row of the statistics
#pragma unroll
    for (int i = 0; i < kFoldQ; i++) {
      const int q = lane + 64 * i;
      st[i] = wave < M && q < (K >> 2) ? reinterpret_cast<const float4 *>(a.fold.x + (size_t)wave * K)[q]
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
#pragma unroll
  for (int gi = 0; gi < kFewMaxGw; gi++) {
    if (gi >= gw || ks * kFewWaves * gw + kFewWaves * gi + wave >= G) break;  // wave-uniform
    floatx16 P[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) P[j][e] = 0.0f;
#pragma unroll
    for (int kp = 0; kp < 2; kp++)
#pragma unroll
      for (int sub = 0; sub < 2; sub++) {
        const f16x8 ah = __builtin_bit_cast(f16x8, xa[gi][0][kp][sub]);
        const f16x8 al = __builtin_bit_cast(f16x8, xa[gi][1][kp][sub]);
#pragma unroll
        for (int j = 0; j < 2; j++) {
          u32x4 b;
          if constexpr (BITS == 8) {
            const uint32_t w0 = cq[gi][j][kp][2 * sub], w1 = cq[gi][j][kp][2 * sub + 1];
            b = u32x4{f16_pair_u8(w0, 0), f16_pair_u8(w0, 16), f16_pair_u8(w1, 0), f16_pair_u8(w1, 16)};
          } else {
            const uint32_t w = cq[gi][j][kp][sub];
            b = u32x4{f16_pair_u4(w, 0), f16_pair_u4(w, 8), f16_pair_u4(w, 16), f16_pair_u4(w, 24)};
          }
          const f16x8 bq = __builtin_bit_cast(f16x8, b);
          P[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bq, P[j], 0, 0, 0);
          P[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bq, P[j], 0, 0, 0);
        }
      }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      float2 sb;
      if constexpr (PT == kParamF16)
        sb = make_float2(half_bits_to_float(pr[gi][j] & 0xffffu), half_bits_to_float(pr[gi][j] >> 16));
      else
        sb = pr[gi][j];
      if constexpr (BITS == 4) sb.y = sb.y - 16.0f * sb.x;
#pragma unroll
      for (int e = 0; e < 4; e++) acc[j][e] = fmaf(sb.x, P[j][e], fmaf(sb.y, gsr[gi][e], acc[j][e]));
    }
  }
  // a batched QKV row's cache position and state (the sequence's control block)
  int ep_pos[kFewEPT], ep_done[kFewEPT];
#pragma unroll
  for (int q = 0; q < kFewEPT; q++) {
    ep_pos[q] = 0;
    ep_done[q] = 0;
    if constexpr (EPI == kEpiQKV)
      if (a.qkv.seqs) {
        ep_pos[q] = ep_sq[q].ctl->valid_len;
        ep_done[q] = ep_sq[q].ctl->done;
      }
  }
  if constexpr (FOLD) {
    {  // rows past M have zero statistics' inputs (mean 0); their results are not stored
      float s1 = 0.0f;
#pragma unroll
      for (int i = 0; i < kFoldQ; i++) s1 += (st[i].x + st[i].y) + (st[i].z + st[i].w);
      const float mean = wave64_sum_dpp(s1) / (float)K;
      float q2 = 0.0f;
#pragma unroll
      for (int i = 0; i < kFoldQ; i++) {
        if (lane + 64 * i < (K >> 2)) {
          const float d0 = st[i].x - mean, d1 = st[i].y - mean, d2 = st[i].z - mean, d3 = st[i].w - mean;
          q2 += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
      }
      const float rstd = 1.0f / sqrtf(wave64_sum_dpp(q2) / (float)K + 1e-5f);
      if (lane == 0) {
        row_mu[wave] = mean;
        row_rs[wave] = rstd;
      }
    }
  }
  // the waves' partials, added in wave order: entry i = (j, e, lane)
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) red[wave][(j * 4 + e) * 64 + lane] = acc[j][e];
  __syncthreads();
  float v[kFewEPT];
#pragma unroll
  for (int q = 0; q < kFewEPT; q++) {
    const int i = tid + 64 * kFewWaves * q;
    float t = red[0][i];
#pragma unroll
    for (int w = 1; w < kFewWaves; w++) t += red[w][i];
    v[q] = t;
  }
  if (S > 1) {
    // the block's 512 partials at ws[(tile, split)], agent-scope stores (coherent across the
    // XCDs' L2s); the last block of the tile adds the splits in split order
    float *wsb = a.ws + (size_t)tn * S * 512;
#pragma unroll
    for (int q = 0; q < kFewEPT; q++)
      __hip_atomic_store(wsb + (size_t)ks * 512 + tid + 64 * kFewWaves * q, v[q], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) last_flag = atomicInc(a.cnt + tn, (uint32_t)(S - 1)) == (uint32_t)(S - 1) ? 1u : 0u;
    __syncthreads();
    if (!last_flag) return;
    // every split's loads issued before the first add
    float w[kFewEPT][kFewMaxSplits];
#pragma unroll
    for (int q = 0; q < kFewEPT; q++)
#pragma unroll
      for (int s2 = 0; s2 < kFewMaxSplits; s2++)
        w[q][s2] = s2 < S && s2 != ks ? __hip_atomic_load(wsb + (size_t)s2 * 512 + tid + 64 * kFewWaves * q,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                      : v[q];
#pragma unroll
    for (int q = 0; q < kFewEPT; q++) {
      float t = w[q][0];
#pragma unroll
      for (int s2 = 1; s2 < kFewMaxSplits; s2++)
        if (s2 < S) t += w[q][s2];
      v[q] = t;
    }
  }
  // entry i -> row m = 4 h + e, column n0 + 32 j + c
  if constexpr (EPI == kEpiGelu) {
#pragma unroll
    for (int q = 0; q < kFewEPT; q++) {
      const int i = tid + 64 * kFewWaves * q, j = i >> 8, e = (i >> 6) & 3, ln = i & 63;
      const int m = 4 * (ln >> 5) + e, cl = 32 * j + (ln & 31), n = n0 + cl;
      const float gv = gelu_tanh_exp(FOLD ? row_rs[m] * (v[q] - row_mu[m] * ep_g[q]) + ep_b[q]
                                      : v[q] + ep_b[q]);  // N is a multiple of 64 here
      gel[m][cl] = gv;
      if (m < M) {
        uint32_t hb, lb;
        split_f16(gv, hb, lb);
        a.xo.hi[(size_t)m * N + n] = (uint16_t)hb;
        a.xo.lo[(size_t)m * N + n] = (uint16_t)lb;
      }
    }
    __syncthreads();
    // per row, the sum of its 64 GELU values in column order (two rows per wave)
#pragma unroll
    for (int r2 = 0; r2 < kFewRows / kFewWaves; r2++) {
      const int m = wave + kFewWaves * r2;
      const float t = wave_sum(gel[m][lane]);
      if (lane == 0 && m < M) a.xo.gs[(size_t)m * (N / kGroup) + tn] = t;
    }
    return;
  } else {
#pragma unroll
    for (int q = 0; q < kFewEPT; q++) {
      const int i = tid + 64 * kFewWaves * q, j = i >> 8, e = (i >> 6) & 3, ln = i & 63;
      const int m = 4 * (ln >> 5) + e, n = n0 + 32 * j + (ln & 31);
      if (m >= M || n >= N) continue;
      const float val = FOLD ? row_rs[m] * (v[q] - row_mu[m] * ep_g[q]) + ep_b[q] : v[q] + ep_b[q];
      if constexpr (EPI == kEpiStore) {
        a.y[(size_t)m * N + n] = val;
      } else if constexpr (EPI == kEpiResid) {
        a.y[(size_t)m * N + n] = ep_y[q] + val;
      } else {
        const int d = a.qkv.d_model;
        if (n < d) {
          a.qkv.q_out[(size_t)m * d + n] = val;
        } else {
          const int idx = n < 2 * d ? n - d : n - 2 * d;
          const int hh = idx >> 6, e2 = idx & 63;
          void *cache = n < 2 * d ? a.qkv.k_cache : a.qkv.v_cache;
          int pos = a.qkv.pos0 + m;
          if (a.qkv.seqs) {  // batched decode: row m is sequence m
            if (ep_done[q]) continue;
            pos = ep_pos[q];
            cache = static_cast<char *>(n < 2 * d ? ep_sq[q].k : ep_sq[q].v) +
                    a.qkv.layer_off * (KVT == kKvBf16 ? 2 : 4);
          }
          const size_t ci = ((size_t)hh * a.qkv.max_seq + pos) * kHeadDim + e2;
          if constexpr (KVT == kKvBf16) {
            static_cast<uint16_t *>(cache)[ci] = (uint16_t)float_to_bf16_bits(val);
          } else {
            static_cast<float *>(cache)[ci] = val;
          }
        }
      }
    }
  }
}

// fp32 rows [M][K] -> hi/lo fp16 planes and per-group row sums; one wave per 64-group
__global__ __launch_bounds__(256) void split_rows_kernel(const float *x, int M, int K, SplitOut o) {
  const int G = K / kGroup;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= M * G) return;
  const int m = item / G, g = item % G;
  const size_t i = (size_t)m * K + g * kGroup + lane;
  const float v = x[i];
  uint32_t h, l;
  split_f16(v, h, l);
  o.hi[i] = (uint16_t)h;
  o.lo[i] = (uint16_t)l;
  const float s = wave_sum(v);
  if (lane == 0) o.gs[(size_t)m * G + g] = s;
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

// Tile configurations: small (64 x 64, two blocks per CU) for the prefill of one
// utterance, large (128 x 128, one block per CU) for many rows.
constexpr int kStages = 3;

struct Plan {
  int TM, TN, mode, nN, mt, S, gps, blocks;
  size_t lds;
};

template <int BITS, int PT, int TM, int TN>
constexpr size_t lds_bytes() {
  return (size_t)kStages * Shape<BITS, PT, TM, TN>::STAGE;
}

Plan make_plan(const GemmArgs &a, int bits, int ptype) {
  Plan p{};
  const bool large = a.M > kGemmSmallTileRows;
  p.TM = p.TN = large ? 2 : 1;
  const int BM = 64 * p.TM, BN = 64 * p.TN;
  const int G = a.ql.K / kGroup;
  p.nN = (a.ql.N + BN - 1) / BN;
  p.mt = (a.M + BM - 1) / BM;
  const int tiles = p.nN * p.mt;
  const int slots = std::max(1, a.n_cu) * (large ? 1 : 2);
  // Split count with the lowest modelled time; partial tiles must fit the workspace.
  // Small tiles (copier waves, two blocks per CU), in microseconds, fitted to MI355X timings
  // of the decoder's four GEMM shapes at 8, 99, 163 and 235 rows: ~0.95 us per split (the
  // last block of a tile adds every partial), and per K group of a block ~0.42 us while the
  // blocks fit one per CU, rising with the blocks per CU.  Large tiles (one block per CU):
  // rounds x (groups + fill) in group units plus a reduction term.
  int bestS = 1;
  double best = 1e30;
  for (int S = 1; S <= std::min(G, 32); S++) {
    const int gps = (G + S - 1) / S, Se = (G + gps - 1) / gps;
    if (Se != S) continue;
    if (S > 1 && ((size_t)tiles * S * BM * BN > a.ws_floats || tiles > a.cnt_words)) break;
    const int blocks = tiles * S;
    const int rounds = (blocks + slots - 1) / slots;
    double cost;
    if (large) {
      cost = rounds * (gps + 3) + (S > 1 ? 2 : 0);
    } else {
      const double per_cu = (double)blocks / std::max(1, a.n_cu);
      cost = 0.953 * S - 1.044 * gps * rounds + 1.462 * gps * std::max(1.0, per_cu);
    }
    if (cost < best) {
      best = cost;
      bestS = S;
    }
  }
  p.S = bestS;
  p.gps = (G + p.S - 1) / p.S;
  p.mode = p.mt <= 4 ? 1 : 0;
  p.blocks = p.mode == 1 ? ((p.nN * p.S + 7) / 8) * 8 * p.mt : tiles * p.S;
  (void)bits;
  (void)ptype;
  return p;
}

template <int BITS, int PT, int EPI, int KVT, int TM, int TN>
hipError_t set_cfg_attr() {
  return hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_kernel<BITS, PT, EPI, KVT, TM, TN, kStages, true>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes<BITS, PT, TM, TN>());
}

template <int BITS, int PT, int EPI, int KVT, int TM, int TN>
hipError_t launch_cfg(const GemmArgs &a, const Plan &p, hipStream_t s) {
  // large tiles (one block per CU) run with copier waves; small tiles keep two blocks per CU
  constexpr bool prod = true;
  auto *fn = gemm_kernel<BITS, PT, EPI, KVT, TM, TN, kStages, prod>;
  constexpr size_t lds = lds_bytes<BITS, PT, TM, TN>();
  hipLaunchKernelGGL(fn, dim3(p.blocks), dim3(prod ? 512 : 256), lds, s, a, p.mode, p.nN, p.mt, p.S, p.gps);
  return hipGetLastError();
}

template <int BITS, int PT>
hipError_t init_bits() {
  hipError_t e = hipSuccess;
  auto chk = [&](hipError_t x) {
    if (e == hipSuccess) e = x;
  };
  chk(set_cfg_attr<BITS, PT, kEpiStore, 0, 1, 1>());
  chk(set_cfg_attr<BITS, PT, kEpiStore, 0, 2, 2>());
  chk(set_cfg_attr<BITS, PT, kEpiResid, 0, 1, 1>());
  chk(set_cfg_attr<BITS, PT, kEpiResid, 0, 2, 2>());
  chk(set_cfg_attr<BITS, PT, kEpiGelu, 0, 1, 1>());
  chk(set_cfg_attr<BITS, PT, kEpiGelu, 0, 2, 2>());
  chk(set_cfg_attr<BITS, PT, kEpiQKV, kKvBf16, 1, 1>());
  chk(set_cfg_attr<BITS, PT, kEpiQKV, kKvBf16, 2, 2>());
  chk(set_cfg_attr<BITS, PT, kEpiQKV, kKvF32, 1, 1>());
  chk(set_cfg_attr<BITS, PT, kEpiQKV, kKvF32, 2, 2>());
  return e;
}

template <int BITS, int PT, int EPI, int KVT>
hipError_t launch_epi(const GemmArgs &a, const Plan &p, hipStream_t s) {
  if (p.TM == 2) return launch_cfg<BITS, PT, EPI, KVT, 2, 2>(a, p, s);
  return launch_cfg<BITS, PT, EPI, KVT, 1, 1>(a, p, s);
}

template <int BITS, int PT>
hipError_t gemm_dispatch(const GemmArgs &a, const Plan &p, int epi, int kvt, hipStream_t s) {
  switch (epi) {
    case kEpiStore:
      return launch_epi<BITS, PT, kEpiStore, 0>(a, p, s);
    case kEpiResid:
      return launch_epi<BITS, PT, kEpiResid, 0>(a, p, s);
    case kEpiGelu:
      return launch_epi<BITS, PT, kEpiGelu, 0>(a, p, s);
    case kEpiQKV:
      return kvt == kKvBf16 ? launch_epi<BITS, PT, kEpiQKV, kKvBf16>(a, p, s)
                            : launch_epi<BITS, PT, kEpiQKV, kKvF32>(a, p, s);
    default:
      return hipErrorInvalidValue;
  }
}

template <int BITS, int PT, int EPI, int KVT, bool FOLD = false>
hipError_t few_launch(const GemmArgs &a, int nN, int S, int gw, hipStream_t s) {
  hipLaunchKernelGGL((few_kernel<BITS, PT, EPI, KVT, FOLD>), dim3(nN * S), dim3(64 * kFewWaves), 0, s, a, nN, S,
                     gw);
  return hipGetLastError();
}

template <int BITS, int PT>
hipError_t few_dispatch(const GemmArgs &a, int nN, int S, int gw, int epi, int kvt, hipStream_t s) {
  switch (epi) {
    case kEpiStore:
      return few_launch<BITS, PT, kEpiStore, 0>(a, nN, S, gw, s);
    case kEpiResid:
      return few_launch<BITS, PT, kEpiResid, 0>(a, nN, S, gw, s);
    case kEpiGelu:
      return a.fold.x ? few_launch<BITS, PT, kEpiGelu, 0, true>(a, nN, S, gw, s)
                      : few_launch<BITS, PT, kEpiGelu, 0>(a, nN, S, gw, s);
    case kEpiQKV:
      if (a.fold.x)
        return kvt == kKvBf16 ? few_launch<BITS, PT, kEpiQKV, kKvBf16, true>(a, nN, S, gw, s)
                              : few_launch<BITS, PT, kEpiQKV, kKvF32, true>(a, nN, S, gw, s);
      return kvt == kKvBf16 ? few_launch<BITS, PT, kEpiQKV, kKvBf16>(a, nN, S, gw, s)
                            : few_launch<BITS, PT, kEpiQKV, kKvF32>(a, nN, S, gw, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t gemm_init() {
  hipError_t e = init_bits<8, kParamF16>();
  if (e == hipSuccess) e = init_bits<8, kParamF32>();
  if (e == hipSuccess) e = init_bits<4, kParamF16>();
  if (e == hipSuccess) e = init_bits<4, kParamF32>();
  return e;
}

size_t gemm_ws_floats(int n_cu) {
  // split-K is only chosen while tiles x splits stay within about two rounds of blocks
  return (size_t)4 * std::max(1, n_cu) * 64 * 64 * 4;
}

hipError_t launch_gemm(const GemmArgs &a, int bits, int ptype, int epi, int kvt, hipStream_t s) {
  if (a.ql.K % kGroup != 0 || a.M <= 0 || a.ql.N <= 0) return hipErrorInvalidValue;
  if (epi == kEpiGelu && a.ql.N % kGroup != 0) return hipErrorInvalidValue;
  if (a.fold.x) {  // the folded LayerNorm: few-row products with one group a wave only
    if (a.M > kFewRows || (bits != 8 && bits != 4) || a.ql.K % 256 != 0 || a.ql.K > 256 * kFoldQ ||
        (epi != kEpiQKV && epi != kEpiGelu) || !a.fold.gamma || !a.fold.G || !a.fold.c)
      return hipErrorInvalidValue;
  }
  if (a.tfi.st && ((epi != kEpiQKV && epi != kEpiGelu) || a.ql.K > 32 * kGroup || !a.tfi.G || !a.tfi.c || a.fold.x))
    return hipErrorInvalidValue;
  if (a.tfo.st && (epi != kEpiResid || a.ql.N % kGroup != 0 || !a.tfo.gamma || !a.tfo.o.hi || !a.tfo.o.lo ||
                   !a.tfo.o.gs || a.fold.x))
    return hipErrorInvalidValue;
  // (the tiled folds are written for the tiled product only)
  if (a.M <= kFewRows && (bits == 8 || bits == 4) && !a.tfi.st && !a.tfo.st) {
    // a group per wave while that keeps the splits within kFewMaxSplits (gw > kFewMaxGw
    // beyond that: the tiled GEMM)
    const int nN = (a.ql.N + 63) / 64, G = a.ql.K / kGroup;
    const int gw = (G + kFewWaves * kFewMaxSplits - 1) / (kFewWaves * kFewMaxSplits);
    const int S = (G + kFewWaves * gw - 1) / (kFewWaves * gw);
    const bool ws_ok = S == 1 || (a.ws && a.cnt && (size_t)nN * S * 512 <= a.ws_floats && nN <= a.cnt_words);
    if (a.fold.x && (!ws_ok || gw != 1)) return hipErrorInvalidValue;
    if (ws_ok && gw <= kFewMaxGw) {
      if (bits == 8)
        return ptype == kParamF16 ? few_dispatch<8, kParamF16>(a, nN, S, gw, epi, kvt, s)
                                  : few_dispatch<8, kParamF32>(a, nN, S, gw, epi, kvt, s);
      return ptype == kParamF16 ? few_dispatch<4, kParamF16>(a, nN, S, gw, epi, kvt, s)
                                : few_dispatch<4, kParamF32>(a, nN, S, gw, epi, kvt, s);
    }
  }
  const Plan p = make_plan(a, bits, ptype);
  if (p.S > 1 && (a.ws == nullptr || a.cnt == nullptr)) return hipErrorInvalidValue;
  if (bits == 8) {
    return ptype == kParamF16 ? gemm_dispatch<8, kParamF16>(a, p, epi, kvt, s)
                              : gemm_dispatch<8, kParamF32>(a, p, epi, kvt, s);
  }
  if (bits == 4) {
    return ptype == kParamF16 ? gemm_dispatch<4, kParamF16>(a, p, epi, kvt, s)
                              : gemm_dispatch<4, kParamF32>(a, p, epi, kvt, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_split_rows(const float *x, int M, int K, const SplitOut &o, hipStream_t s) {
  if (K % kGroup != 0 || M <= 0) return hipErrorInvalidValue;
  const int items = M * (K / kGroup);
  hipLaunchKernelGGL(split_rows_kernel, dim3((items + 3) / 4), dim3(256), 0, s, x, M, K, o);
  return hipGetLastError();
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
