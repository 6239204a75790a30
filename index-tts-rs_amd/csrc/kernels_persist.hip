// Persistent decode step for gfx950: one cooperative launch runs a whole decode step
// (embedding, every block, ln_f + final_norm + mel_head) on one block per CU.
//
// Why persistent.  A batch-1 step is a chain of ~120 dependent GEMV/attention phases over
// small matrices.  As separate kernels each phase pays the launch floor (~2 us) plus the
// loaded HBM latency (~1.7 us) before its first weight byte arrives.  Here every block
// keeps its share of each phase's weights in registers and prefetches the next layer's
// share as soon as the current one is consumed, so HBM latency overlaps the dependency
// chain; what is left per phase is the exchange of the phase's output vector.
//
// Exchange.  Every cross-block value travels as one 64-bit word (epoch << 32 | fp32 bits)
// written and read with device-scope relaxed atomics: a reader polls the words it needs
// until each carries the phase's epoch, so no fence or grid barrier is needed and a stale
// word is never mistaken for a fresh one.  Epoch of (step s, layer l, phase p):
// s * 8 * (n_layer + 1) + 8 * l + p + 1, with s from the control block.
//
// Waves.  Waves 0-1 ("pollers") poll exchange words into LDS; waves 2-7 ("compute") hold
// the weights.  Vector loads complete in issue order per wave, so a wave with prefetches
// in flight would not see a poll result before its prefetches land: the roles never mix.
// All waves meet at __syncthreads, which on gfx950 waits for LDS traffic only.
//
// Ownership.  For a matrix with N rows, block b owns rows [N*b/B, N*(b+1)/B).  A block's
// rows of c_proj and of the MLP's c_proj coincide, so it keeps its slice of the residual
// stream locally.  Attention: block b < H*S serves head b/S over key split b%S; the last
// split of a head to finish (device-scope counter) combines the head's partials.
//
// Every wait is bounded: a timed-out poller raises the error word, and every block leaves
// at its next barrier.
#include <algorithm>

#include "kernels.h"

namespace itts {

namespace {

// 512 threads: with two waves per SIMD each wave may hold 256 registers, room for two
// matrices' weight slices plus a poll batch.
constexpr int kThreads = 512;
constexpr int kPollThreads = 128;     // waves 0-1
constexpr int kComputeThreads = 384;  // waves 2-7
constexpr int kComputeWaves = kComputeThreads / 64;
constexpr int kKeySlots = kComputeThreads / 8;  // attention: 8 lanes per key
constexpr int kKeyPasses = 4;                   // keys per split <= kKeySlots * kKeyPasses
constexpr int kPollBatch = 20;        // exchange words per poller thread in flight
constexpr int kPollSpan = kPollThreads * kPollBatch;
static_assert(kPollSpan <= kPersistPad, "exchange padding must cover one poll batch");
constexpr long kSpinLimit = 1L << 21;
// 16-byte code chunks per compute lane (rows per block x chunks per row / 384, rounded
// up) for the full-size decoder on 256 blocks
constexpr int kSlQkv = 4, kSlProj = 2, kSlFc = 5, kSlMp = 5, kSlHead = 7;

struct RowMap {
  int row0, rows, C;  // first row, row count, 16-byte chunks per row
};

__device__ inline RowMap rows_of(int N, int C, int b, int B) {
  const int r0 = (int)((long)N * b / B), r1 = (int)((long)N * (b + 1) / B);
  return RowMap{r0, r1 - r0, C};
}

__device__ inline void ll_store(uint64_t *p, uint32_t ep, float v) {
  __hip_atomic_store(p, ((uint64_t)ep << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ll_load(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld_u32(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Pollers: read n exchange words of epoch ep into dst (LDS).  False on timeout or when
// another block raised the error word.  src must stay readable for kPollSpan words past
// n: the exchange arrays carry that much padding, so the loads need no clamping.
__device__ bool poll_words(const uint64_t *src, int n, uint32_t ep, float *dst, uint32_t *err) {
  const int t = threadIdx.x;
  for (int base = 0; base < n; base += kPollSpan) {
    const int lim = n - base - t;  // word k of this lane is in range when 128k < lim
    uint64_t w[kPollBatch];
    long spins = 0;
    while (true) {
      // lane offset made opaque per spin: the compiler keeps one base register instead of
      // hoisting a 64-bit address per word (per call site) out of the loops
      uint32_t to = (uint32_t)(base + t) * 8u;
      asm volatile("" : "+v"(to));
      const uint64_t *p = reinterpret_cast<const uint64_t *>(reinterpret_cast<const char *>(src) + to);
#pragma unroll
      for (int k = 0; k < kPollBatch; k++) w[k] = ll_load(p + k * kPollThreads);
      bool all = true;
#pragma unroll
      for (int k = 0; k < kPollBatch; k++) all = all && (kPollThreads * k >= lim || (uint32_t)(w[k] >> 32) == ep);
      if (__all(all)) break;
      if (++spins > kSpinLimit) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
      if ((spins & 63) == 0 && ld_u32(err) != 0) return false;
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int k = 0; k < kPollBatch; k++)
      if (kPollThreads * k < lim) dst[base + t + kPollThreads * k] = __uint_as_float((uint32_t)w[k]);
  }
  return true;
}

// (scale, bias) of one group as held in registers: fp16x2 in one register, or float2.
template <int PT>
struct ParamReg {
  using type = float2;
};
template <>
struct ParamReg<kParamF16> {
  using type = uint32_t;
};
__device__ inline float2 param_value(uint32_t w) {
  return make_float2(half_bits_to_float(w & 0xffffu), half_bits_to_float(w >> 16));
}
__device__ inline float2 param_value(float2 p) { return p; }

template <int PT, int NS>
struct Slots {
  uint4 c[NS];
  typename ParamReg<PT>::type p[NS];
};

// Compute lane cl (0..383) loads its chunks of the block's rows of ql (int8 codes).
// The rows are contiguous and a row is C = K/16 chunks, so chunk c of the block sits at
// codes + row0*K + 16c and its group parameters at params[row0*K/64 + c/4].
template <int PT, int NS>
__device__ inline void load_slots(Slots<PT, NS> &s, const DevQL &ql, const RowMap &m, int cl) {
  using P = typename ParamReg<PT>::type;
  const int total = m.rows * m.C;
  const char *cb = reinterpret_cast<const char *>(ql.codes + (size_t)m.row0 * ql.K);
  const char *pb = reinterpret_cast<const char *>(static_cast<const P *>(ql.params) + (size_t)m.row0 * (ql.K / kGroup));
  // uniform base + 32-bit lane offset (a block's slice is far below 4 GiB)
  uint32_t lo = (uint32_t)cl;
  asm volatile("" : "+v"(lo));
#pragma unroll
  for (int j = 0; j < NS; j++) {
    const uint32_t c = lo + (uint32_t)(kComputeThreads * j);
    if ((int)c < total) {
      s.c[j] = *reinterpret_cast<const uint4 *>(cb + c * 16u);
      s.p[j] = *reinterpret_cast<const P *>(pb + (c >> 2) * (uint32_t)sizeof(P));
    }
  }
}

__device__ inline float dot16(const uint4 c, const float *xc) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 xv = *reinterpret_cast<const float4 *>(xc + 4 * i);
    acc += xv.x * (float)(w[i] & 0xffu);
    acc += xv.y * (float)((w[i] >> 8) & 0xffu);
    acc += xv.z * (float)((w[i] >> 16) & 0xffu);
    acc += xv.w * (float)(w[i] >> 24);
  }
  return acc;
}

// Compute lanes: per-chunk partial products into part[] (LDS).
template <int PT, int NS>
__device__ inline void dot_slots(const Slots<PT, NS> &s, const RowMap &m, const float *xn, const float *xsum,
                                 float *part, int cl) {
  const int total = m.rows * m.C;
#pragma unroll
  for (int j = 0; j < NS; j++) {
    const int c = cl + kComputeThreads * j;
    if (c < total) {
      const int kc = c % m.C;
      const float2 p = param_value(s.p[j]);
      part[c] = p.x * dot16(s.c[j], xn + kc * 16) + p.y * xsum[kc];
    }
    // one chunk's activations in registers at a time
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Compute wave cw sums rows cw, cw+6, ... of part[] in a fixed order; lane 0 receives
// the row value with its bias and calls epi(row_in_block, value).
template <class Epi>
__device__ inline void row_sums(const RowMap &m, const float *part, const float *bias, int cw, int lane, Epi epi) {
  for (int r = cw; r < m.rows; r += kComputeWaves) {
    float acc = 0.0f;
    for (int c = lane; c < m.C; c += 64) acc += part[r * m.C + c];
    acc = wave_sum(acc);
    if (lane == 0) epi(r, acc + bias[m.row0 + r]);
  }
}

__device__ inline void chunk_sums(const float *x, int n, float *xsum) {
  for (int c = threadIdx.x; c < n / 16; c += kThreads) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += x[c * 16 + i];
    xsum[c] = s;
  }
}

struct PersistShared {
  float red[16];
  int abort;
  int last;
  float m_w[kComputeWaves], l_w[kComputeWaves];
};

template <int PT>
__global__ __launch_bounds__(kThreads) void decode_persist_kernel(PersistArgs a) {
  __shared__ PersistShared sh;
  extern __shared__ float lds[];
  DecodeCtl *ctl = a.ctl;
  if (ctl->done) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bool poller = tid < kPollThreads;
  const int cl = tid - kPollThreads;           // compute lane (when !poller)
  const int cw = wave - kPollThreads / 64;     // compute wave (when !poller)
  const int B = gridDim.x, b = blockIdx.x;
  const int d = a.d, F = a.F, V = a.V, H = a.H, S = a.S;
  const int tok = ctl->tok, pos = ctl->pos, vlen = ctl->valid_len;
  const uint32_t xstep = (uint32_t)ctl->xstep;
  const uint32_t ep0 = xstep * a.ep_stride + 1u;
  const int L = vlen + 1;  // keys including the row this step appends
  uint32_t *err = a.err;

  // LDS: xin[xin_len] | xn[d] | xsum[xin_len/16] | part[part_len] | own[own_len] |
  //      own_mid[own_len] | qs[64] | kn[64] | vn[64] | ow[12*64] | pp[S*66]
  float *xin = lds;
  float *xn = xin + a.xin_len;
  float *xsum = xn + d;
  float *part = xsum + a.xin_len / 16;
  float *own = part + a.part_len;
  float *own_mid = own + a.own_len;
  float *qs = own_mid + a.own_len;
  float *kn = qs + 64;
  float *vn = kn + 64;
  float *ow = vn + 64;
  float *pp = ow + kComputeWaves * 64;

  const RowMap m_qkv = rows_of(3 * d, d / 16, b, B);
  const RowMap m_proj = rows_of(d, d / 16, b, B);
  const RowMap m_fc = rows_of(F, d / 16, b, B);
  const RowMap m_mp = rows_of(d, F / 16, b, B);
  const RowMap m_head = rows_of(V, d / 16, b, B);
  const bool attn_block = b < H * S;
  const int ah = b / S, aj = b % S;
  const int j0 = (int)((long)L * aj / S), j1 = (int)((long)L * (aj + 1) / S);
  const int kslot = cl >> 3, dsl = cl & 7;     // attention lane: key slot, 8-dim slice

  if (tid == 0) {
    sh.abort = 0;
    sh.last = 0;
  }

  // ---- prologue: layer 0's weights in flight; the step embedding -------------------
  Slots<PT, kSlQkv> wq;
  Slots<PT, kSlProj> wp;
  Slots<PT, kSlFc> wf;
  Slots<PT, kSlMp> wm;
  if (!poller) {
    const DevLayer &L0 = a.layers[0];
    load_slots<PT>(wq, L0.attn, m_qkv, cl);
    load_slots<PT>(wp, L0.proj, m_proj, cl);
  }
  for (int i = tid; i < d; i += kThreads) xin[i] = a.mel_emb[(size_t)tok * d + i] + a.mel_pos[(size_t)pos * d + i];
  __syncthreads();
  for (int r = tid; r < m_proj.rows; r += kThreads) own[r] = xin[m_proj.row0 + r];

  for (int l = 0; l < a.n_layer; l++) {
    const DevLayer &Ly = a.layers[l];
    const uint32_t ep = ep0 + (uint32_t)l * 8u;
    // ---------------- P1: LN1, QKV rows; K/V rows into the cache --------------------
    if (l > 0) {
      if (poller && !poll_words(a.x_x, d, ep - 8u + 6u, xin, err)) sh.abort = 1;
      __syncthreads();
      if (sh.abort) return;
    }
    layernorm_lds_inplace_to<kThreads>(xin, xn, Ly.ln1_w, Ly.ln1_b, d, sh.red);
    chunk_sums(xn, d, xsum);
    __syncthreads();
    if (!poller) {
      dot_slots(wq, m_qkv, xn, xsum, part, cl);
      load_slots<PT>(wf, Ly.fc, m_fc, cl);
    }
    __syncthreads();
    if (!poller) {
      row_sums(m_qkv, part, Ly.attn.bias, cw, lane, [&](int r, float v) {
        const int R = m_qkv.row0 + r;
        ll_store(a.x_qkv + R, ep + 1u, v);
        if (R >= d) {
          const int idx = R < 2 * d ? R - d : R - 2 * d;
          const int h = idx >> 6, e = idx & 63;
          uint16_t *cache = static_cast<uint16_t *>(R < 2 * d ? a.kc : a.vc);
          cache[(((size_t)l * H + h) * a.max_seq + vlen) * 64 + e] = (uint16_t)float_to_bf16_bits(v);
        }
      });
    }
    // ---------------- P2: attention split of head ah over keys [j0, j1) ----------------
    if (attn_block) {
      // K/V of the split's cached rows (the appended row comes from the exchange);
      // loaded before waiting for the query
      uint4 kreg[kKeyPasses], vreg[kKeyPasses];
      if (!poller) {
        const size_t hb = ((size_t)l * H + ah) * a.max_seq * 64;
        const uint16_t *kh = static_cast<const uint16_t *>(a.kc) + hb;
        const uint16_t *vh = static_cast<const uint16_t *>(a.vc) + hb;
#pragma unroll
        for (int ps = 0; ps < kKeyPasses; ps++) {
          const int key = j0 + kslot + kKeySlots * ps;
          if (key < j1 && key < L - 1) {
            kreg[ps] = *reinterpret_cast<const uint4 *>(kh + (size_t)key * 64 + dsl * 8);
            vreg[ps] = *reinterpret_cast<const uint4 *>(vh + (size_t)key * 64 + dsl * 8);
          } else {
            kreg[ps] = make_uint4(0, 0, 0, 0);
            vreg[ps] = make_uint4(0, 0, 0, 0);
          }
        }
      }
      if (poller) {
        bool ok = poll_words(a.x_qkv + ah * 64, 64, ep + 1u, qs, err);
        if (ok && j1 == L) {  // this split holds the appended row
          ok = poll_words(a.x_qkv + d + ah * 64, 64, ep + 1u, kn, err) &&
               poll_words(a.x_qkv + 2 * d + ah * 64, 64, ep + 1u, vn, err);
        }
        if (!ok) sh.abort = 1;
      }
      __syncthreads();
      if (sh.abort) return;
      // the appended row as the cache stores it (bf16)
      if (tid < 64) {
        kn[tid] = bf16_bits_to_float(float_to_bf16_bits(kn[tid]));
        vn[tid] = bf16_bits_to_float(float_to_bf16_bits(vn[tid]));
      }
      __syncthreads();
      float sc[kKeyPasses];
      if (!poller) {
        float mloc = -INFINITY;
#pragma unroll
        for (int ps = 0; ps < kKeyPasses; ps++) {
          const int key = j0 + kslot + kKeySlots * ps;
          float pd = 0.0f;
          if (key < j1) {
            if (key == L - 1) {
#pragma unroll
              for (int e = 0; e < 8; e++) pd += qs[dsl * 8 + e] * kn[dsl * 8 + e];
            } else {
              const uint32_t w[4] = {kreg[ps].x, kreg[ps].y, kreg[ps].z, kreg[ps].w};
#pragma unroll
              for (int e = 0; e < 4; e++) {
                pd += qs[dsl * 8 + 2 * e] * __uint_as_float(w[e] << 16);
                pd += qs[dsl * 8 + 2 * e + 1] * __uint_as_float(w[e] & 0xffff0000u);
              }
            }
          }
          pd += __shfl_xor(pd, 1, 64);
          pd += __shfl_xor(pd, 2, 64);
          pd += __shfl_xor(pd, 4, 64);
          sc[ps] = key < j1 ? pd * 0.125f : -INFINITY;
          mloc = fmaxf(mloc, sc[ps]);
        }
        mloc = wave_max(mloc);
        if (lane == 0) sh.m_w[cw] = mloc;
      }
      __syncthreads();
      float M = -INFINITY;
      for (int w = 0; w < kComputeWaves; w++) M = fmaxf(M, sh.m_w[w]);
      if (!poller) {
        float o8[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o8[e] = 0.0f;
        float lsum = 0.0f;
#pragma unroll
        for (int ps = 0; ps < kKeyPasses; ps++) {
          const int key = j0 + kslot + kKeySlots * ps;
          if (key < j1) {
            const float p = __expf(sc[ps] - M);
            if (dsl == 0) lsum += p;
            if (key == L - 1) {
#pragma unroll
              for (int e = 0; e < 8; e++) o8[e] += p * vn[dsl * 8 + e];
            } else {
              const uint32_t w[4] = {vreg[ps].x, vreg[ps].y, vreg[ps].z, vreg[ps].w};
#pragma unroll
              for (int e = 0; e < 4; e++) {
                o8[2 * e] += p * __uint_as_float(w[e] << 16);
                o8[2 * e + 1] += p * __uint_as_float(w[e] & 0xffff0000u);
              }
            }
          }
        }
        lsum = wave_sum(lsum);
#pragma unroll
        for (int off = 8; off < 64; off <<= 1) {
#pragma unroll
          for (int e = 0; e < 8; e++) o8[e] += __shfl_xor(o8[e], off, 64);
        }
        if (lane < 8) {
#pragma unroll
          for (int e = 0; e < 8; e++) ow[cw * 64 + lane * 8 + e] = o8[e];
        }
        if (lane == 0) sh.l_w[cw] = lsum;
      }
      __syncthreads();
      // block partial -> exchange; the last split of the head to finish combines
      if (tid < 64) {
        float osum = 0.0f;
        for (int w = 0; w < kComputeWaves; w++) osum += ow[w * 64 + tid];
        uint64_t *pw = a.x_part + ((size_t)ah * S + aj) * 66;
        ll_store(pw + 2 + tid, ep + 2u, osum);
        if (tid == 0) {
          float lt = 0.0f;
          for (int w = 0; w < kComputeWaves; w++) lt += sh.l_w[w];
          ll_store(pw, ep + 2u, M);
          ll_store(pw + 1, ep + 2u, lt);
          // wrapping device-scope counter: cycles 0..S-1, so the S-th arrival reads S-1
          const uint32_t old = atomicInc(a.cnt + ah * kCntStride, (uint32_t)(S - 1));
          sh.last = old == (uint32_t)(S - 1);
        }
      }
      __syncthreads();
      if (sh.last) {
        if (poller && !poll_words(a.x_part + (size_t)ah * S * 66, S * 66, ep + 2u, pp, err)) sh.abort = 1;
        __syncthreads();
        if (sh.abort) return;
        if (tid < 64) {
          float Mg = -INFINITY;
          for (int s = 0; s < S; s++) Mg = fmaxf(Mg, pp[s * 66]);
          float den = 0.0f, num = 0.0f;
          for (int s = 0; s < S; s++) {
            if (pp[s * 66] == -INFINITY) continue;
            const float f = __expf(pp[s * 66] - Mg);
            den += pp[s * 66 + 1] * f;
            num += pp[s * 66 + 2 + tid] * f;
          }
          ll_store(a.x_attn + ah * 64 + tid, ep + 3u, num / den);
        }
      }
    }
    // ---------------- P3: c_proj rows + residual ------------------------------------
    if (poller && !poll_words(a.x_attn, d, ep + 3u, xin, err)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    chunk_sums(xin, d, xsum);
    __syncthreads();
    if (!poller) {
      dot_slots(wp, m_proj, xin, xsum, part, cl);
      load_slots<PT>(wm, Ly.mproj, m_mp, cl);
    }
    __syncthreads();
    if (!poller) {
      row_sums(m_proj, part, Ly.proj.bias, cw, lane, [&](int r, float v) {
        const float xm = own[r] + v;
        own_mid[r] = xm;
        ll_store(a.x_mid + m_proj.row0 + r, ep + 4u, xm);
      });
    }
    // ---------------- P4: LN2, c_fc rows + GELU ------------------------------------
    if (poller && !poll_words(a.x_mid, d, ep + 4u, xin, err)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    layernorm_lds_inplace_to<kThreads>(xin, xn, Ly.ln2_w, Ly.ln2_b, d, sh.red);
    chunk_sums(xn, d, xsum);
    __syncthreads();
    if (!poller) {
      dot_slots(wf, m_fc, xn, xsum, part, cl);
      if (l + 1 < a.n_layer) load_slots<PT>(wq, a.layers[l + 1].attn, m_qkv, cl);
    }
    __syncthreads();
    if (!poller) {
      row_sums(m_fc, part, Ly.fc.bias, cw, lane,
               [&](int r, float v) { ll_store(a.x_f + m_fc.row0 + r, ep + 5u, gelu_tanh(v)); });
    }
    // ---------------- P5: mlp c_proj rows + residual ---------------------------------
    if (poller && !poll_words(a.x_f, F, ep + 5u, xin, err)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    chunk_sums(xin, F, xsum);
    __syncthreads();
    if (!poller) {
      dot_slots(wm, m_mp, xin, xsum, part, cl);
      if (l + 1 < a.n_layer) load_slots<PT>(wp, a.layers[l + 1].proj, m_proj, cl);
    }
    __syncthreads();
    if (!poller) {
      row_sums(m_mp, part, Ly.mproj.bias, cw, lane, [&](int r, float v) {
        const float xo = own_mid[r] + v;
        own[r] = xo;
        ll_store(a.x_x + m_mp.row0 + r, ep + 6u, xo);
      });
    }
  }
  // ---------------- head: ln_f, final_norm, mel_head rows -> logits ------------------
  {
    Slots<PT, kSlHead> wh;
    if (!poller) load_slots<PT>(wh, a.head, m_head, cl);
    const uint32_t ep = ep0 + (uint32_t)(a.n_layer - 1) * 8u;
    if (poller && !poll_words(a.x_x, d, ep + 6u, xin, err)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    layernorm_lds_inplace_to<kThreads>(xin, xn, a.ln_f_w, a.ln_f_b, d, sh.red);
    layernorm_lds_inplace<kThreads>(xn, a.fn_w, a.fn_b, d, sh.red);
    chunk_sums(xn, d, xsum);
    __syncthreads();
    if (!poller) dot_slots(wh, m_head, xn, xsum, part, cl);
    __syncthreads();
    if (!poller)
      row_sums(m_head, part, a.head.bias, cw, lane, [&](int r, float v) { a.logits[m_head.row0 + r] = v; });
  }
  // Block 0 closes the step.  Every block read the control block at its start, before its
  // first exchange word, and block 0 gets here only after every block's last exchange.
  if (b == 0 && tid == 0) {
    ctl->valid_len = vlen + 1;
    ctl->xstep = (int32_t)(xstep + 1u);
  }
}

}  // namespace

bool persist_supported(int d, int F, int V, int H, int n_layer, int max_seq, int B, int *S_out) {
  if (B < 1 || H < 1 || d % 64 != 0 || F % 64 != 0 || n_layer < 1) return false;
  const int S = std::min(12, B / H);
  if (S < 1) return false;
  if ((max_seq + S - 1) / S > kKeySlots * kKeyPasses) return false;
  auto fits = [&](int N, int C, int slots) {
    return (long)((N + B - 1) / B) * C <= (long)slots * kComputeThreads;
  };
  if (!fits(3 * d, d / 16, kSlQkv) || !fits(d, d / 16, kSlProj) || !fits(F, d / 16, kSlFc) ||
      !fits(d, F / 16, kSlMp) || !fits(V, d / 16, kSlHead))
    return false;
  *S_out = S;
  return true;
}

size_t persist_lds_bytes(const PersistArgs &a) {
  const size_t f = (size_t)a.xin_len + a.d + a.xin_len / 16 + a.part_len + 2 * (size_t)a.own_len + 3 * 64 +
                   kComputeWaves * 64 + (size_t)a.S * 66;
  return f * sizeof(float);
}

hipError_t launch_decode_persist(PersistArgs a, int ptype, hipStream_t s) {
  void *args[] = {&a};
  const size_t lds = persist_lds_bytes(a);
  const void *fn = ptype == kParamF16 ? reinterpret_cast<const void *>(decode_persist_kernel<kParamF16>)
                                      : reinterpret_cast<const void *>(decode_persist_kernel<kParamF32>);
  return hipLaunchCooperativeKernel(fn, dim3(a.B), dim3(kThreads), args, (unsigned)lds, s);
}

hipError_t persist_init() {
  for (const void *fn : {reinterpret_cast<const void *>(decode_persist_kernel<kParamF16>),
                         reinterpret_cast<const void *>(decode_persist_kernel<kParamF32>)}) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPersistMaxLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t persist_blocks_per_cu(int ptype, size_t lds, int *blocks) {
  const void *fn = ptype == kParamF16 ? reinterpret_cast<const void *>(decode_persist_kernel<kParamF16>)
                                      : reinterpret_cast<const void *>(decode_persist_kernel<kParamF32>);
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, fn, kThreads, lds);
}

}  // namespace itts
