// Persistent decode step for gfx950: one launch of one block per CU runs a whole decode step
// (embedding, every block, ln_f + final_norm + mel_head) on one block per CU.
//
// Why persistent.  A batch-1 step is a chain of ~120 dependent GEMV/attention phases over
// small matrices.  As separate kernels each phase pays the launch floor (~2 us) plus the
// loaded HBM latency (~1.7 us) before its first weight byte arrives.  Here every block
// keeps its share of each matrix in registers, loaded ahead of use, so HBM latency
// overlaps the dependency chain; what is left per phase is the exchange of the phase's
// output vector between blocks.
//
// Exchange.  Values travel in 16-byte words: three fp32 values and the epoch's low bits in
// each 8-byte half (xstore), written by one lane with one store and read with one load,
// both device-coherent.  A reader polls the words it needs until both halves of each carry
// the phase's epoch, so no fence or grid barrier is needed and a stale (or partly stale)
// word is never taken for a fresh one.  A producer's values form one
// segment of ceil(len/3) words.  Epoch of (step s, layer l, phase p):
// s * 8 * (n_layer + 1) + 8 * l + p + 1, with s from the control block.  A word is
// rewritten only after every block has consumed it: the next write of any array depends
// on every block's output of a later phase.
//
// Wave roles.  Vector memory operations of one wave complete in issue order (stores
// included), and the compiler waits for them by count.  So that no wave ever waits for
// an unrelated operation, each wave kind issues one kind of global access:
//   pollers  (waves 0-5)  : loads only - exchange polls, the embedding;
//   publisher (wave 6)    : exchange words, K/V cache rows and logits (stores), and the
//                           next layer's parameters (LDS-DMA copies it waits for where it
//                           has slack);
//   loaders  (waves 7-15) : loads only, all unconditional - the weight slices (ahead of
//                           use) and the attention K/V rows (LDS-DMA); they compute the
//                           dot products and row sums in LDS.
// Each role is its own instantiation of the step program (run<BITS, PT, ROLE>), all executing
// the same sequence of __syncthreads, which on gfx950 waits for LDS traffic only.
//
// Ownership.  For a matrix with N rows, block b owns rows [N*b/B, N*(b+1)/B).  A block's
// rows of c_proj and of the MLP's c_proj coincide, so it keeps its slice of the residual
// stream in LDS.  Attention: block b < H*S serves head b/S over key split b%S; the last
// split of a head to finish (device-scope counter) combines the head's partials.
//
// Every wait is bounded: a timed-out poller raises the error word, and every block leaves
// at its next barrier.
#include <algorithm>

#include "kernels.h"

namespace itts {

namespace {

constexpr int kThreads = 1024;
constexpr int kPollWaves = 6;
constexpr int kPollThreads = kPollWaves * 64;  // waves 0-5
constexpr int kPubWave = 6;
constexpr int kLoadWave0 = 7;
constexpr int kLoadWaves = 9;
constexpr int kLoadThreads = kLoadWaves * 64;  // waves 7-15
constexpr int kKeySlots = kLoadThreads / 8;    // attention: 8 lanes per key
constexpr int kKeyPasses = 3;                  // keys per split <= kKeySlots * kKeyPasses
constexpr long kSpinLimit = 1L << 21;
constexpr int kPartVals = 66;                  // attention partial: max, denominator, 64 outputs
constexpr int kPartWords = (kPartVals + 2) / 3;
constexpr int kHeadWords = (64 + 2) / 3;
// 16-byte code chunks per loader lane (rows per block x chunks per row / 576, rounded up)
// for the full-size decoder on 256 blocks
constexpr int kSlQkv = 3, kSlProj = 1, kSlFc = 3, kSlMp = 3, kSlHead = 5;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct RowMap {
  int row0, rows, C;  // first row, row count, 16-byte chunks per row (K/16 int8, K/32 int4)
};

__device__ inline int row_start(int N, int b, int B) { return (int)((long)N * b / B); }
__device__ inline RowMap rows_of(int N, int C, int b, int B) {
  const int r0 = row_start(N, b, B);
  return RowMap{r0, row_start(N, b + 1, B) - r0, C};
}
// The block whose rows contain row r: the largest b with row_start(N, b, B) <= r.
__device__ inline int block_of(int N, int r, int B) { return (int)(((long)(r + 1) * B - 1) / N); }
__device__ inline int words_for(int n) { return (n + 2) / 3; }

// Activation rows as the dot products read them: every 16-byte code chunk's EPC values (16
// int8 or 32 int4 codes) followed by 4 floats of padding.  Loader lanes take consecutive
// chunks, so without the padding a wave's float4 reads would sit 64 (128) bytes apart and
// fall into a quarter (an eighth) of the LDS banks; 80 (144) bytes apart, 16 consecutive
// lanes cover every bank once.  Value k of a row sits at xpad(k).
template <int BITS>
__device__ inline int xpad(int k) {
  return k + ((k >> (BITS == 8 ? 4 : 5)) << 2);
}
// i / d for 0 <= i < 2^16 and 1 <= d <= 2^15: one multiply-high by m = floor((2^32-1)/d) + 1.
// i*m/2^32 exceeds i/d by i*(m - 2^32/d)/2^32 < i/2^32, below the 1/d gap to the next
// integer for these ranges, so the floor is exact.
// d == 1 would need m = 2^32: it is kept as m = 0 and divides by returning i.
struct FastDiv {
  uint32_t m;
  __device__ explicit FastDiv(int d) : m(d == 1 ? 0u : 0xffffffffu / (uint32_t)d + 1u) {}
  __device__ int operator()(int i) const { return m ? (int)__umulhi((uint32_t)i, m) : i; }
};

__device__ inline uint32_t ld_u32(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Load through the global address space.  Pointers read from the layer table are generic
// to the compiler, and a generic (flat) load also counts against the LDS wait counter, so
// every LDS wait of a wave would wait for its weight prefetches too.
template <class T>
__device__ inline T gld(const void *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}
// The same as a non-temporal load (the nt cache policy): the weights stream through once
// per step, and marked so they disturb the caches the exchange words pass through less
// (a decode step measured 595 us against 608 us with plain loads).
template <class T>
__device__ inline T gld_nt(const void *p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) T *)p);
}

// ---- exchange words --------------------------------------------------------------------
// A word holds three values and the epoch's low 16 bits twice, once in each 8-byte half:
//   dword 0: a | dword 1: c bits 0-15, epoch bits 16-31 | dword 2: b | dword 3: c bits
//   16-31, epoch bits 16-31.
// No AMD document promises that a 16-byte store is observed whole by a 16-byte load (the
// memory model's single-copy atomicity stops at 64 bits, for aligned 8-byte accesses), so
// each half carries the epoch and a reader takes a word only when both halves do: a load
// that saw one half of an older word fails and is polled again.  A word is rewritten at
// most 200 epochs (one step) after it was last written, so 16 bits tell the expected epoch
// from any earlier one; epochs restart at 1 when the exchange memory is cleared.
__device__ inline uint32_t xtag(uint32_t ep) { return ep << 16; }
__device__ inline bool xword_ok(const u32x4 w, uint32_t tag) { return ((w.y ^ tag) | (w.w ^ tag)) < 0x10000u; }
// (a, b, c, 0) of a word that checked.
__device__ inline u32x4 xword_vals(const u32x4 w) { return u32x4{w.x, w.z, (w.y & 0xffffu) | (w.w << 16), 0u}; }
// One device-coherent 16-byte store of values a, b, c at epoch ep.
__device__ inline void xstore(u32x4 *p, float a, float b, float c, uint32_t ep) {
  const uint32_t uc = __float_as_uint(c), tag = xtag(ep);
  const u32x4 v = {__float_as_uint(a), (uc & 0xffffu) | tag, __float_as_uint(b), (uc >> 16) | tag};
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}

// K device-coherent 16-byte loads in flight together, then one wait: the loads are issued
// in one asm block so that the results are read only after the wait.
template <int K>
__device__ inline void xload(u32x4 (&w)[K], const u32x4 *const (&p)[K]);
template <>
__device__ inline void xload<1>(u32x4 (&w)[1], const u32x4 *const (&p)[1]) {
  asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=&v"(w[0]) : "v"(p[0]) : "memory");
}
template <>
__device__ inline void xload<2>(u32x4 (&w)[2], const u32x4 *const (&p)[2]) {
  asm volatile(
      "global_load_dwordx4 %0, %2, off sc1\n\t"
      "global_load_dwordx4 %1, %3, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1])
      : "v"(p[0]), "v"(p[1])
      : "memory");
}
template <>
__device__ inline void xload<5>(u32x4 (&w)[5], const u32x4 *const (&p)[5]) {
  asm volatile(
      "global_load_dwordx4 %0, %5, off sc1\n\t"
      "global_load_dwordx4 %1, %6, off sc1\n\t"
      "global_load_dwordx4 %2, %7, off sc1\n\t"
      "global_load_dwordx4 %3, %8, off sc1\n\t"
      "global_load_dwordx4 %4, %9, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4])
      : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4])
      : "memory");
}

// Pollers: wait until the nw words at addr(0..nw-1) carry epoch ep, then hand each to
// put(i, word).  K words per poller lane per pass; a lane past nw re-reads a word in range
// and ignores it.  False on timeout or when another block raised the error word.
template <int K, class Addr, class Put>
__device__ __forceinline__ bool poll_k(int nw, uint32_t ep, uint32_t *err, int t, Addr addr, Put put) {
  for (int base = 0; base < nw; base += K * kPollThreads) {
    const u32x4 *p[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
      const int i = base + t + k * kPollThreads;
      p[k] = addr(i < nw ? i : base);
    }
    u32x4 w[K];
    const uint32_t tag = xtag(ep);
    long spins = 0;
    while (true) {
      xload<K>(w, p);
      bool all = true;
#pragma unroll
      for (int k = 0; k < K; k++)  // bitwise, not short-circuit: no branch per word
        all = all & ((base + t + k * kPollThreads >= nw) | xword_ok(w[k], tag));
      if (__all(all)) break;
      if (++spins > kSpinLimit) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
      if ((spins & 63) == 0 && ld_u32(err) != 0) return false;
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
      const int i = base + t + k * kPollThreads;
      if (i < nw) put(i, xword_vals(w[k]));
    }
  }
  return true;
}

template <class Addr, class Put>
__device__ __forceinline__ bool poll(int nw, uint32_t ep, uint32_t *err, int t, Addr addr, Put put) {
  if (nw <= kPollThreads) return poll_k<1>(nw, ep, err, t, addr, put);
  if (nw <= 2 * kPollThreads) return poll_k<2>(nw, ep, err, t, addr, put);
  return poll_k<5>(nw, ep, err, t, addr, put);
}

// Word j of a segment holding len values (starting at value 0) scattered to dst.
__device__ inline void put_word(float *dst, int j, int len, u32x4 v) {
  const int e0 = 3 * j;
  if (e0 < len) dst[e0] = __uint_as_float(v.x);
  if (e0 + 1 < len) dst[e0 + 1] = __uint_as_float(v.y);
  if (e0 + 2 < len) dst[e0 + 2] = __uint_as_float(v.z);
}

// Pollers: the whole N-vector published by blocks (block s's rows as one segment of W
// words) into dst, in row order or (PAD) in the dot products' padded layout; rs[s] =
// row_start(N, s, B) for s in [0, B] (LDS table).
template <int BITS, bool PAD>
__device__ __forceinline__ bool poll_rows(const void *arr, int N, int B, const int *rs, uint32_t ep, float *dst,
                                          uint32_t *err, int t) {
  const int W = words_for((N + B - 1) / B);
  const FastDiv divW(W);
  const u32x4 *src = static_cast<const u32x4 *>(arr);
  return poll(
      B * W, ep, err, t, [&](int i) { return src + i; },
      [&](int i, u32x4 v) {
        const int s = divW(i), j = i - s * W;
        const int r0 = rs[s], len = rs[s + 1] - r0;
        const float f[3] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z)};
#pragma unroll
        for (int e = 0; e < 3; e++) {
          const int k = r0 + 3 * j + e;
          if (3 * j + e < len) dst[PAD ? xpad<BITS>(k) : k] = f[e];
        }
      });
}

// Pollers: poll_rows for the input of a folded LayerNorm: x into dst in row order and
// gamma * x (gamma in LDS) into dst_g in the dot products' padded layout.
template <int BITS>
__device__ __forceinline__ bool poll_rows_ln(const void *arr, int N, int B, const int *rs, uint32_t ep, float *dst,
                                             float *dst_g, const float *gamma, uint32_t *err, int t) {
  const int W = words_for((N + B - 1) / B);
  const FastDiv divW(W);
  const u32x4 *src = static_cast<const u32x4 *>(arr);
  return poll(
      B * W, ep, err, t, [&](int i) { return src + i; },
      [&](int i, u32x4 v) {
        const int s = divW(i), j = i - s * W;
        const int r0 = rs[s], len = rs[s + 1] - r0;
        const float f[3] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z)};
#pragma unroll
        for (int e = 0; e < 3; e++) {
          const int k = 3 * j + e;
          if (k < len) {
            dst[r0 + k] = f[e];
            dst_g[xpad<BITS>(r0 + k)] = gamma[r0 + k] * f[e];
          }
        }
      });
}

// Publisher lane j < W: the block's rows (vals[0..rows)) as its segment of arr.
__device__ inline void publish_rows(void *arr, int N, int B, int b, const float *vals, int rows, uint32_t ep,
                                    int lane) {
  const int W = words_for((N + B - 1) / B);
  if (lane < W) {
    const int e0 = 3 * lane;
    xstore(static_cast<u32x4 *>(arr) + b * W + lane, e0 < rows ? vals[e0] : 0.0f, e0 + 1 < rows ? vals[e0 + 1] : 0.0f,
           e0 + 2 < rows ? vals[e0 + 2] : 0.0f, ep);
  }
}

// ---- weights -----------------------------------------------------------------------
// (scale, bias) of one group as held in registers: fp16x2 in one register, or float2.
template <int PT>
struct ParamReg {
  using type = f32x2;
};
template <>
struct ParamReg<kParamF16> {
  using type = uint32_t;
};
__device__ inline float2 param_value(uint32_t w) {
  return make_float2(half_bits_to_float(w & 0xffffu), half_bits_to_float(w >> 16));
}
__device__ inline float2 param_value(f32x2 p) { return make_float2(p.x, p.y); }

template <int PT, int NS>
struct Slots {
  u32x4 c[NS];
  typename ParamReg<PT>::type p[NS];
};

// Loader lane ll (0..575) loads its chunks of the block's rows of ql.  The rows are
// contiguous and a row is C 16-byte chunks (16 int8 or 32 int4 codes), so chunk c of the
// block sits at codes + row0*K*BITS/8 + 16c with its group parameters at
// params[row0*K/64 + c/(64/codes per chunk)].  Every load is issued (a chunk past the
// block's share reads chunk 0 instead, row row0 < N always exists), so the number of loads
// in flight is the same on every path.
template <int BITS, int PT, int NS>
__device__ inline void load_slots(Slots<PT, NS> &s, const DevQL &ql, const RowMap &m, int ll) {
  using P = typename ParamReg<PT>::type;
  constexpr uint32_t kGroupShift = BITS == 8 ? 2 : 1;  // chunks per group: 4 or 2
  const int total = m.rows * m.C;
  const char *cb = reinterpret_cast<const char *>(ql.codes + (size_t)m.row0 * ql.K * BITS / 8);
  const char *pb = reinterpret_cast<const char *>(static_cast<const P *>(ql.params) + (size_t)m.row0 * (ql.K / kGroup));
  uint32_t lo = (uint32_t)ll;
  asm volatile("" : "+v"(lo));
#pragma unroll
  for (int j = 0; j < NS; j++) {
    uint32_t c = lo + (uint32_t)(kLoadThreads * j);
    c = (int)c < total ? c : 0u;
    s.c[j] = gld_nt<u32x4>(cb + c * 16u);
    s.p[j] = gld_nt<P>(pb + (c >> kGroupShift) * (uint32_t)sizeof(P));
  }
}

// 32 4-bit codes (low nibble first) against 32 activations: (sum of code*x, sum of x).
__device__ inline float2 dot32(const u32x4 c, const float *xc) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float acc = 0.0f, xs = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 xa = *reinterpret_cast<const float4 *>(xc + 8 * i);
    const float4 xb = *reinterpret_cast<const float4 *>(xc + 8 * i + 4);
    // even and odd nibbles as bytes, so that each code converts with one byte-select
    // conversion (the same values, summed in the same order)
    uint32_t lo = w[i] & 0x0f0f0f0fu, hi = (w[i] >> 4) & 0x0f0f0f0fu;
    asm("" : "+v"(lo), "+v"(hi));  // opaque: otherwise folded back into one bit-field extract per code
    acc += xa.x * (float)(lo & 0xffu);
    acc += xa.y * (float)(hi & 0xffu);
    acc += xa.z * (float)((lo >> 8) & 0xffu);
    acc += xa.w * (float)((hi >> 8) & 0xffu);
    acc += xb.x * (float)((lo >> 16) & 0xffu);
    acc += xb.y * (float)((hi >> 16) & 0xffu);
    acc += xb.z * (float)(lo >> 24);
    acc += xb.w * (float)(hi >> 24);
    xs += ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
  }
  return make_float2(acc, xs);
}

// 16 codes against 16 activations: (sum of code*x, sum of x).
__device__ inline float2 dot16(const u32x4 c, const float *xc) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float acc = 0.0f, xs = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 xv = *reinterpret_cast<const float4 *>(xc + 4 * i);
    acc += xv.x * (float)(w[i] & 0xffu);
    acc += xv.y * (float)((w[i] >> 8) & 0xffu);
    acc += xv.z * (float)((w[i] >> 16) & 0xffu);
    acc += xv.w * (float)(w[i] >> 24);
    xs += (xv.x + xv.y) + (xv.z + xv.w);
  }
  return make_float2(acc, xs);
}

// Loaders: per-chunk partial products into part[] (LDS): scale * sum(code*x) + bias *
// sum(x), the group affine folded per 16-value chunk; xn in the padded layout (xpad).
template <int BITS, int PT, int NS>
__device__ inline void dot_slots(const Slots<PT, NS> &s, const RowMap &m, const float *xn, float *part, int ll) {
  const int total = m.rows * m.C;
  // per-slot chunk indices are recomputed per call rather than hoisted out of the layer
  // loop (they would hold a register per slot and matrix for the whole step)
  uint32_t lo = (uint32_t)ll;
  asm volatile("" : "+v"(lo));
#pragma unroll
  for (int j = 0; j < NS; j++) {
    const int c = (int)lo + kLoadThreads * j;
    if (c < total) {
      const int kc = c % m.C;
      const float2 p = param_value(s.p[j]);
      const float2 r = BITS == 8 ? dot16(s.c[j], xn + kc * 20) : dot32(s.c[j], xn + kc * 36);
      part[c] = p.x * r.x + p.y * r.y;
    }
    // one chunk's activations in registers at a time
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---- cross-lane reductions ---------------------------------------------------------------
// DPP (ALU row shifts and broadcasts, no LDS round trip).  They need every lane of the wave
// active.  Fixed order, so every block reduces identically.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ inline float dpp_f(float v, float old) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}
// Inclusive scan within each row of 16 lanes: lane 15 of a row holds the row's sum.
__device__ inline float row16_sum(float x) {
  x += dpp_f<0x111, 0xf, 0xf>(x, 0.0f);  // row_shr:1
  x += dpp_f<0x112, 0xf, 0xf>(x, 0.0f);  // row_shr:2
  x += dpp_f<0x114, 0xf, 0xe>(x, 0.0f);  // row_shr:4, lanes 4-15
  x += dpp_f<0x118, 0xf, 0xc>(x, 0.0f);  // row_shr:8, lanes 8-15
  return x;
}
// Sum over the wave, returned to every lane.
__device__ inline float wave64_sum(float x) {
  x = row16_sum(x);
  x += dpp_f<0x142, 0xa, 0xf>(x, 0.0f);  // row_bcast:15 into rows 1, 3
  x += dpp_f<0x143, 0xc, 0xf>(x, 0.0f);  // row_bcast:31 into rows 2, 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}
// Max over the wave, returned to every lane.
__device__ inline float wave64_max(float x) {
  const float ni = -INFINITY;
  x = fmaxf(x, dpp_f<0x111, 0xf, 0xf>(x, ni));
  x = fmaxf(x, dpp_f<0x112, 0xf, 0xf>(x, ni));
  x = fmaxf(x, dpp_f<0x114, 0xf, 0xe>(x, ni));
  x = fmaxf(x, dpp_f<0x118, 0xf, 0xc>(x, ni));
  x = fmaxf(x, dpp_f<0x142, 0xa, 0xf>(x, ni));
  x = fmaxf(x, dpp_f<0x143, 0xc, 0xf>(x, ni));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// Loader waves sum the rows of part[] (a row is m.C chunk partials), in a fixed order:
// rows of 256 chunks or more take a wave each (lane 0 calls epi), shorter rows 16 lanes
// each, four rows per wave, rows lw*4.. of each pass of 9 waves (the last lane of a row
// calls epi).  epi(row, sum) receives the row's product without its bias.
template <class Epi>
__device__ inline void row_sums(const RowMap &m, const float *part, int lw, int lane, Epi epi) {
  if (m.C >= 256) {  // long rows: a wave per row
    for (int r = lw; r < m.rows; r += kLoadWaves) {
      float acc = 0.0f;
      for (int c = lane; c < m.C; c += 64) acc += part[r * m.C + c];
      acc = wave64_sum(acc);
      if (lane == 0) epi(r, acc);
    }
    return;
  }
  const int sub = lane >> 4, sl = lane & 15;
  for (int r0 = lw * 4; r0 < m.rows; r0 += kLoadWaves * 4) {
    const int r = r0 + sub;
    float acc = 0.0f;
    if (r < m.rows)
      for (int c = sl; c < m.C; c += 16) acc += part[r * m.C + c];
    acc = row16_sum(acc);
    if (sl == 15 && r < m.rows) epi(r, acc);
  }
}

// ---- folded LayerNorm statistics ---------------------------------------------------------
// Pollers, beside the other waves' products: mean and rstd of the LDS row x (n values, a
// multiple of 4, at most 4 * kPollThreads; biased variance, eps 1e-5, gpt.rs:339,375) into
// st[24], st[25].  Poller wave w holds values 256w .. 256w + 255 (one float4 a lane) and
// writes their sum, mean and sum of squared deviations from that mean (two passes over
// registers) to st[w], st[8 + w], st[16 + w]; the last wave to finish (a wrapping LDS
// counter, zero between uses) merges them in wave order: mean = sum / n, and the squared
// deviations from it are each wave's own plus count * (wave mean - mean)^2 (the parallel
// form of the two-pass variance, Chan, Golub and LeVeque 1979).
__device__ __forceinline__ void ln_stats(const float *x, int n, float *st, uint32_t *cnt, int t) {
  const int nq = n >> 2, nw = (nq + 63) >> 6, w = t >> 6, lane = t & 63;
  if (w >= nw) return;  // wave-uniform
  const bool act = t < nq;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (act) v = reinterpret_cast<const float4 *>(x)[t];
  const float sum = wave64_sum((v.x + v.y) + (v.z + v.w));
  const float m = sum / (float)(4 * min(64, nq - w * 64));
  float q = 0.0f;
  if (act) {
    const float d0 = v.x - m, d1 = v.y - m, d2 = v.z - m, d3 = v.w - m;
    q = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
  }
  q = wave64_sum(q);
  uint32_t old = 0;
  if (lane == 0) {
    st[w] = sum;
    st[8 + w] = m;
    st[16 + w] = q;
    // a wave's LDS operations complete in order: the partials land before the count
    old = atomicInc(cnt, (uint32_t)(nw - 1));
  }
  if (__builtin_amdgcn_readfirstlane(old) != (uint32_t)(nw - 1)) return;
  float s = 0.0f;
  for (int i = 0; i < nw; i++) s += st[i];
  const float mean = s / (float)n;
  float m2 = 0.0f;
  for (int i = 0; i < nw; i++) {
    const float dm = st[8 + i] - mean;
    m2 += st[16 + i] + (float)(4 * min(64, nq - 64 * i)) * (dm * dm);
  }
  if (lane == 0) {
    st[24] = mean;
    st[25] = 1.0f / sqrtf(m2 / (float)n + 1e-5f);
  }
}

// ---- parameters -----------------------------------------------------------------------
// Stages one layer's parameters into a parameter buffer with LDS-DMA copies issued by one
// wave (lane in [0, 64)): no registers are written, and nothing waits for the copies until
// the wave's own s_waitcnt, placed where the wave has slack.  d is a multiple of 64.
// Layer l: [ln_1 gamma d][ln_2 gamma d] and the block's rows of c_qkv, G_qkv, the c_proj
// bias, c_fc, G_fc and the mlp c_proj bias (folded LayerNorms: the betas live in c).
// l == n_layer (the head): [ln_f w][ln_f b][final_norm w][final_norm b][mel_head bias rows].
// Global -> LDS copies issued by hand (lane l's bytes land at lds + l * size, lds in M0).
// Issued with the builtin, every copy waited for the one before it to land: the compiler
// cannot tell apart the LDS bytes a pending copy writes and waits for it before the next
// access to LDS, the next copy included.  The publisher's own s_waitcnt covers them before
// their LDS rows are read.  M0 is set before every copy (and declared clobbered).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void pub_dma16(const void *src, const float *lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void pub_dma4(const void *src, const float *lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ void stage_params_dma(const PersistArgs &a, int l, float *lp, const RowMap &mq,
                                                 const RowMap &mp, const RowMap &mf, const RowMap &mm,
                                                 const RowMap &mh, int lane) {
  const int d = a.d;
  const bool head = l >= a.n_layer;
  // the layer's pointers by scalar loads (the constant address space): by vector loads
  // the copies' own source pointers would wait for every copy issued before them, since
  // vector loads complete in issue order
  typedef const __attribute__((address_space(4))) DevLayer ConstLayer;
  ConstLayer *Ly = head ? nullptr : (ConstLayer *)(a.layers) + l;
  const int nv = head ? 4 : 2;
#pragma unroll
  for (int arr = 0; arr < 4; arr++) {
    if (arr >= nv) break;
    const float *src = head ? (arr == 0 ? a.ln_f_w : arr == 1 ? a.ln_f_b : arr == 2 ? a.fn_w : a.fn_b)
                            : (arr == 0 ? Ly->ln1_w : Ly->ln2_w);
    for (int off = 0; off < d; off += 256)  // 64 lanes x 4 floats per copy
      if (off + lane * 4 < d) pub_dma16(src + off + lane * 4, lp + arr * d + off);
  }
  float *bl = lp + nv * d;
  auto rows = [&](const RowMap &m, const float *v) {
    for (int r0 = 0; r0 < m.rows; r0 += 64)
      if (r0 + lane < m.rows) pub_dma4(v + m.row0 + r0 + lane, bl + r0);
    bl += m.rows;
  };
  if (head) {
    rows(mh, a.head.bias);
    return;
  }
  const float *fo = a.fold + fold_floats(d, a.F) * l;
  rows(mq, fo + 3 * d);          // c_qkv
  rows(mq, fo);                  // G_qkv
  rows(mp, Ly->proj.bias);
  rows(mf, fo + 6 * d + a.F);    // c_fc
  rows(mf, fo + 6 * d);          // G_fc
  rows(mm, Ly->mproj.bias);
}

// LayerNorm (biased variance, eps 1e-5) of the LDS row x into the LDS row y (y may be x),
// w and b in LDS (16-byte aligned, n a multiple of 4, n <= 4 * 1024); red holds 32 floats.
// Thread t < n/4 holds values 4t..4t+3 of x, w and b, read with one 16-byte LDS load each,
// all three issued together, so the row is read once and every later pass works from
// registers.  The waves holding values form the sums; every wave adds the wave sums in the
// same order.
// With q4 > 0, y is written in the dot products' padded layout (a float4 of padding after
// every 2^q4 float4s) instead of row order; y may still be x, since every thread reads its
// values before the first barrier and writes after the second.
__device__ __forceinline__ void layer_norm(const float *x, float *y, const float *w, const float *b, int n, float *red,
                                           int tid, int q4 = 0) {
  const int nq = n >> 2, nwv = (nq + 63) >> 6;
  const bool act = tid < nq, wact = tid < nwv * 64;
  float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f), wv = xv, bv = xv;
  if (act) {
    xv = reinterpret_cast<const float4 *>(x)[tid];
    wv = reinterpret_cast<const float4 *>(w)[tid];
    bv = reinterpret_cast<const float4 *>(b)[tid];
  }
  if (wact) {
    const float s = wave64_sum((xv.x + xv.y) + (xv.z + xv.w));
    if ((tid & 63) == 0) red[tid >> 6] = s;
  }
  __syncthreads();
  float mean = 0.0f;
  if (wact) {
    float t = 0.0f;
    for (int i = 0; i < nwv; i++) t += red[i];
    mean = t / (float)n;
    float q = 0.0f;
    if (act) {
      const float d0 = xv.x - mean, d1 = xv.y - mean, d2 = xv.z - mean, d3 = xv.w - mean;
      q = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
    q = wave64_sum(q);
    if ((tid & 63) == 0) red[16 + (tid >> 6)] = q;
  }
  __syncthreads();
  if (act) {
    float t = 0.0f;
    for (int i = 0; i < nwv; i++) t += red[16 + i];
    const float rstd = 1.0f / sqrtf(t / (float)n + 1e-5f);
    float4 yv;
    yv.x = (xv.x - mean) * rstd * wv.x + bv.x;
    yv.y = (xv.y - mean) * rstd * wv.y + bv.y;
    yv.z = (xv.z - mean) * rstd * wv.z + bv.z;
    yv.w = (xv.w - mean) * rstd * wv.w + bv.w;
    reinterpret_cast<float4 *>(y)[q4 > 0 ? tid + (tid >> q4) : tid] = yv;
  }
  __syncthreads();
}

struct __attribute__((aligned(16))) PersistShared {
  float red[32];
  int abort;
  int last;
  uint32_t stat_cnt;  // folded LayerNorm statistics: waves done (wraps to 0)
  float m_w[kLoadWaves], l_w[kLoadWaves];
};

enum Role : int { kRolePoll = 0, kRolePub = 1, kRoleLoad = 2 };

// The whole step as seen by one wave role.  The three instantiations execute the same
// sequence of __syncthreads; each contains only its role's work, so the compiler allocates
// registers per role (a role branch on a divergent condition would be linearised and make
// every wave hold the registers of all roles).
template <int BITS, int PT, int KVF, int ROLE>
__device__ __forceinline__ void run(const PersistArgs &a, PersistShared &sh, float *lds) {
  constexpr bool poller = ROLE == kRolePoll, pub = ROLE == kRolePub, loader = ROLE == kRoleLoad;
  DecodeCtl *ctl = a.ctl;
  const int tid = threadIdx.x, lane = tid & 63;
  const int ll = tid - kLoadWave0 * 64;                                   // loader lane
  const int lw = __builtin_amdgcn_readfirstlane((tid >> 6) - kLoadWave0);  // loader wave
  const int B = gridDim.x, b = blockIdx.x;
  const int d = a.d, F = a.F, H = a.H, S = a.S;
  const int tok = ctl->tok, pos = ctl->pos, vlen = ctl->valid_len;
  const uint32_t xstep = (uint32_t)ctl->xstep;
  const uint32_t ep0 = xstep * a.ep_stride + 1u;
  const int L = vlen + 1;  // keys including the row this step appends
  uint32_t *err = a.err;
  u32x4 *x_part = static_cast<u32x4 *>(a.x_part);
  u32x4 *x_attn = static_cast<u32x4 *>(a.x_attn);

  // LDS (floats): xin[xin_len] | xn[xn_len] | part[part_len] | own[own_len] | own_mid[own_len] |
  // out[out_len] | qs[64] | kn[64] | vn[64] | pp[S*66] | lp[2][lp_len] | kvs[2*3*576*4] |
  // rs[3][B+1] (int); the host rounds every length to a multiple of 4
  float *xin = lds;
  float *xn = xin + a.xin_len;
  float *part = xn + a.xn_len;
  float *own = part + a.part_len;
  float *own_mid = own + a.own_len;
  float *out = own_mid + a.own_len;
  float *qs = out + a.out_len;
  float *kn = qs + 64;
  float *vn = kn + 64;
  float *pp = vn + 64;
  float *lpb = pp + a.pp_len;
  float *kvs = lpb + 2 * a.lp_len;  // [2][kKeyPasses][576] x 16 bytes
  // row_start tables of the by-block exchange arrays: N = d, 3d, F; B + 1 entries each
  int *rs_d = reinterpret_cast<int *>(kvs + 2 * kKeyPasses * kLoadThreads * 4);
  int *rs_3d = rs_d + (B + 1);
  int *rs_f = rs_3d + (B + 1);

  constexpr int EPC = BITS == 8 ? 16 : 32;  // codes per 16-byte chunk
  const RowMap m_qkv = rows_of(3 * d, d / EPC, b, B);
  const RowMap m_proj = rows_of(d, d / EPC, b, B);
  const RowMap m_fc = rows_of(F, d / EPC, b, B);
  const RowMap m_mp = rows_of(d, F / EPC, b, B);
  const RowMap m_head = rows_of(a.V, d / EPC, b, B);
  // rows inside a layer's parameter buffer (stage_params_dma)
  const int bo_cq = 2 * d, bo_gq = bo_cq + m_qkv.rows, bo_p = bo_gq + m_qkv.rows, bo_cf = bo_p + m_proj.rows,
            bo_gf = bo_cf + m_fc.rows, bo_m = bo_gf + m_fc.rows;
  const bool attn_block = b < H * S;
  const int ah = b / S, aj = b % S;
  const int j0 = (int)((long)L * aj / S), j1 = (int)((long)L * (aj + 1) / S);

  // ---- prologue: layer 0's first two matrices in flight; embedding; parameters -------
  Slots<PT, kSlQkv> wq;
  Slots<PT, kSlProj> wp;
  Slots<PT, kSlFc> wf;
  Slots<PT, kSlMp> wm;
  if (loader) {
    load_slots<BITS, PT>(wq, a.layers[0].attn, m_qkv, ll);
    load_slots<BITS, PT>(wp, a.layers[0].proj, m_proj, ll);
  }
  if (poller) {
    for (int i = tid; i < d; i += kPollThreads)
      xin[i] = gld<float>(a.mel_emb + (size_t)tok * d + i) + gld<float>(a.mel_pos + (size_t)pos * d + i);
  }
  if (pub) {
    stage_params_dma(a, 0, lpb, m_qkv, m_proj, m_fc, m_mp, m_head, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  for (int s2 = tid; s2 <= B; s2 += kThreads) {
    rs_d[s2] = row_start(d, s2, B);
    rs_3d[s2] = row_start(3 * d, s2, B);
    rs_f[s2] = row_start(F, s2, B);
  }
  __syncthreads();
  if (pub)
    for (int r = lane; r < m_proj.rows; r += 64) own[r] = xin[m_proj.row0 + r];

  for (int l = 0; l < a.n_layer; l++) {
    // thread index re-derived opaquely per layer: per-thread LDS addresses are recomputed
    // in each layer instead of being hoisted out of the loop and held for the whole step
    int T = tid;
    asm volatile("" : "+v"(T));
    const int lane = T & 63, ll = T - kLoadWave0 * 64;
    const int kslot = ll >> 3, dsl = ll & 7;  // attention loader lane: key slot, 8-dim slice
    const DevLayer &Ly = a.layers[l];
    const uint32_t ep = ep0 + (uint32_t)l * 8u;
    const float *lp = lpb + (l & 1) * a.lp_len;
    // ---------------- P1: LN1 (folded), QKV rows; K/V rows into the cache ------------
    // The loaders start the product on gamma * x while the pollers form the row's
    // statistics; the row sums apply them: rstd * (sum - mean * G) + c.
    if (l > 0) {
      if (poller && !poll_rows_ln<BITS>(a.x_x, d, B, rs_d, ep - 8u + 6u, xin, xn, lp, err, T)) sh.abort = 1;
    } else if (poller) {
      for (int i = T; i < d; i += kPollThreads) xn[xpad<BITS>(i)] = lp[i] * xin[i];
    }
    __syncthreads();
    if (sh.abort) return;
    if (poller) ln_stats(xin, d, sh.red, &sh.stat_cnt, T);
    if (loader) dot_slots<BITS>(wq, m_qkv, xn, part, ll);
    // this layer's c_proj slice (layer 0's came with the prologue), issued once the QKV dot
    // has its codes: 511.8 against 513.6 us per step with it issued after the previous
    // layer's x publish
    if (loader && l > 0) load_slots<BITS, PT>(wp, Ly.proj, m_proj, ll);
    __syncthreads();
    if (loader) {
      const float mu = sh.red[24], rstd = sh.red[25];
      row_sums(m_qkv, part, lw, lane,
               [&](int r, float v) { out[r] = rstd * (v - mu * lp[bo_gq + r]) + lp[bo_cq + r]; });
    }
    __syncthreads();
    if (pub) {
      publish_rows(a.x_qkv, 3 * d, B, b, out, m_qkv.rows, ep + 1u, lane);
      for (int r = lane; r < m_qkv.rows; r += 64) {
        const int R = m_qkv.row0 + r;
        if (R >= d) {
          const int idx = R < 2 * d ? R - d : R - 2 * d;
          const int h = idx >> 6, e = idx & 63;
          const size_t at = (((size_t)l * H + h) * a.max_seq + vlen) * 64 + e;
          if constexpr (KVF)
            static_cast<float *>(R < 2 * d ? a.kc : a.vc)[at] = out[r];
          else
            static_cast<uint16_t *>(R < 2 * d ? a.kc : a.vc)[at] = (uint16_t)float_to_bf16_bits(out[r]);
        }
      }
    }
    // the next layer's parameters: copied by the publisher (a poller's copies would delay
    // its next poll, which completes in issue order); it waits for them after its P4
    // stores, well before the next layer reads them
    if (pub) stage_params_dma(a, l + 1, lpb + ((l + 1) & 1) * a.lp_len, m_qkv, m_proj, m_fc, m_mp, m_head, lane);
    // ---------------- P2: attention split of head ah over keys [j0, j1) ----------------
    if (attn_block) {
      // cached K/V rows of the split (the appended row comes from the exchange), copied
      // straight into LDS (no registers) before the query arrives.  Wave lw of pass ps
      // holds the split's keys 8c .. 8c+7, c = 9 ps + lw (8 lanes per key, each lane 8
      // dimensions); slots past the split or at the appended row read row 0.  bf16 rows:
      // lane ll of pass ps lands at kvs[(ps*576 + ll)*4], K passes then V passes.  f32 rows
      // (twice the bytes): K in kvs and V in the input-row / normalised-row / partials
      // area, which nothing uses between P1's row sums and P3's all-gather; each 8-key
      // chunk c is two 1 KB halves (dimensions 0-3 and 4-7 of every lane's slice), lane
      // at [(2c + half)*256 + lane*4], and a wave whose keys all lie past the split copies
      // nothing (the V area holds only the chunks a split can reach).
      if (loader) {
        const size_t hb = ((size_t)l * H + ah) * a.max_seq * 64;
#pragma unroll
        for (int ps = 0; ps < kKeyPasses; ps++) {
          const int c = ps * kLoadWaves + lw;
          if (KVF && 8 * c >= j1 - j0) continue;
          int key = j0 + kslot + kKeySlots * ps;
          key = key < j1 && key < L - 1 ? key : 0;
          if constexpr (KVF) {
            const float *kh = static_cast<const float *>(a.kc) + hb + (size_t)key * 64 + dsl * 8;
            const float *vh = static_cast<const float *>(a.vc) + hb + (size_t)key * 64 + dsl * 8;
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
              __builtin_amdgcn_global_load_lds(kh + 4 * hf,
                                               (__attribute__((address_space(3))) void *)(kvs + (2 * c + hf) * 256),
                                               16, 0, 0);
              __builtin_amdgcn_global_load_lds(vh + 4 * hf,
                                               (__attribute__((address_space(3))) void *)(xin + (2 * c + hf) * 256),
                                               16, 0, 0);
            }
          } else {
            const uint16_t *kh = static_cast<const uint16_t *>(a.kc) + hb;
            const uint16_t *vh = static_cast<const uint16_t *>(a.vc) + hb;
            float *wk = kvs + (ps * kLoadThreads + lw * 64) * 4;
            float *wv = kvs + ((kKeyPasses + ps) * kLoadThreads + lw * 64) * 4;
            __builtin_amdgcn_global_load_lds(kh + (size_t)key * 64 + dsl * 8,
                                             (__attribute__((address_space(3))) void *)wk, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vh + (size_t)key * 64 + dsl * 8,
                                             (__attribute__((address_space(3))) void *)wv, 16, 0, 0);
          }
        }
      }
      if (poller) {
        // q (and, for the split holding the appended row, k and v) of head ah: the words
        // of the blocks whose QKV rows cover them, polled together
        const int N3 = 3 * d, Wq = words_for((N3 + B - 1) / B);
        const int *rs3 = rs_3d;
        const bool kv_too = j1 == L;
        const int lq = ah * 64, lk = d + ah * 64, lv = 2 * d + ah * 64;
        const int bq = block_of(N3, lq, B), bk = block_of(N3, lk, B), bv = block_of(N3, lv, B);
        const int nq = (block_of(N3, lq + 63, B) - bq + 1) * Wq;
        const int nk = kv_too ? (block_of(N3, lk + 63, B) - bk + 1) * Wq : 0;
        const int nv = kv_too ? (block_of(N3, lv + 63, B) - bv + 1) * Wq : 0;
        const u32x4 *src = static_cast<const u32x4 *>(a.x_qkv);
        const FastDiv divWq(Wq);
        // word i of the concatenation (q words, then k, then v) -> its group's first block,
        // first row and destination, and its index within the group
        auto group = [&](int i, int &gb, int &lo, float *&dst) {
          if (i < nq) {
            gb = bq, lo = lq, dst = qs;
            return i;
          }
          if (i < nq + nk) {
            gb = bk, lo = lk, dst = kn;
            return i - nq;
          }
          gb = bv, lo = lv, dst = vn;
          return i - nq - nk;
        };
        const bool ok = poll(
            nq + nk + nv, ep + 1u, err, T,
            [&](int i) {
              int gb, lo;
              float *dst;
              const int li = group(i, gb, lo, dst);
              return src + gb * Wq + li;
            },
            [&](int i, u32x4 v) {
              int gb, lo;
              float *dst;
              const int li = group(i, gb, lo, dst);
              const int sq = divWq(li), s = gb + sq, j = li - sq * Wq;
              const int r0 = rs3[s], len = rs3[s + 1] - r0;
              const float f[3] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z)};
#pragma unroll
              for (int e = 0; e < 3; e++) {
                const int rr = r0 + 3 * j + e;
                if (3 * j + e < len && rr >= lo && rr < lo + 64) dst[rr - lo] = f[e];
              }
            });
        if (!ok) sh.abort = 1;
      }
      __syncthreads();
      if (sh.abort) return;
      // the appended row as the cache stores it (bf16 rows round it)
      if (pub && !KVF) {
        kn[lane] = bf16_bits_to_float(float_to_bf16_bits(kn[lane]));
        vn[lane] = bf16_bits_to_float(float_to_bf16_bits(vn[lane]));
      }
      __syncthreads();
      float sc[kKeyPasses];
      if (loader) {
        // the copies above are the loaders' latest vector-memory operations
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        float mloc = -INFINITY;
#pragma unroll
        for (int ps = 0; ps < kKeyPasses; ps++) {
          const int key = j0 + kslot + kKeySlots * ps;
          float pd = 0.0f;
          if (key < j1) {
            if (key == L - 1) {
#pragma unroll
              for (int e = 0; e < 8; e++) pd += qs[dsl * 8 + e] * kn[dsl * 8 + e];
            } else if constexpr (KVF) {
              const int c = ps * kLoadWaves + lw;
              const float4 k0 = *reinterpret_cast<const float4 *>(kvs + 2 * c * 256 + lane * 4);
              const float4 k1 = *reinterpret_cast<const float4 *>(kvs + (2 * c + 1) * 256 + lane * 4);
              const float *qq = qs + dsl * 8;
              pd += qq[0] * k0.x;
              pd += qq[1] * k0.y;
              pd += qq[2] * k0.z;
              pd += qq[3] * k0.w;
              pd += qq[4] * k1.x;
              pd += qq[5] * k1.y;
              pd += qq[6] * k1.z;
              pd += qq[7] * k1.w;
            } else {
              const uint4 kq = *reinterpret_cast<const uint4 *>(kvs + (ps * kLoadThreads + ll) * 4);
              const uint32_t w[4] = {kq.x, kq.y, kq.z, kq.w};
#pragma unroll
              for (int e = 0; e < 4; e++) {
                pd += qs[dsl * 8 + 2 * e] * __uint_as_float(w[e] << 16);
                pd += qs[dsl * 8 + 2 * e + 1] * __uint_as_float(w[e] & 0xffff0000u);
              }
            }
          }
          // sum over the key's 8 lanes, to all 8: xor 1 and 2 within quads, then each quad
          // adds its neighbour quad (row_shr:4 into lanes 4-7 / 12-15, row_shl:4 into 0-3 /
          // 8-11); a + b == b + a, so all 8 lanes hold the same value
          pd += dpp_f<0xB1, 0xf, 0xf>(pd, 0.0f);  // quad_perm [1,0,3,2]
          pd += dpp_f<0x4E, 0xf, 0xf>(pd, 0.0f);  // quad_perm [2,3,0,1]
          pd = pd + dpp_f<0x114, 0xf, 0xa>(pd, 0.0f) + dpp_f<0x104, 0xf, 0x5>(pd, 0.0f);
          sc[ps] = key < j1 ? pd * 0.125f : -INFINITY;
          mloc = fmaxf(mloc, sc[ps]);
        }
        mloc = wave64_max(mloc);
        if (lane == 0) sh.m_w[lw] = mloc;
      }
      __syncthreads();
      float M = -INFINITY;
      for (int w = 0; w < kLoadWaves; w++) M = fmaxf(M, sh.m_w[w]);
      if (loader) {
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
            } else if constexpr (KVF) {
              const int c = ps * kLoadWaves + lw;
              const float4 v0 = *reinterpret_cast<const float4 *>(xin + 2 * c * 256 + lane * 4);
              const float4 v1 = *reinterpret_cast<const float4 *>(xin + (2 * c + 1) * 256 + lane * 4);
              o8[0] += p * v0.x;
              o8[1] += p * v0.y;
              o8[2] += p * v0.z;
              o8[3] += p * v0.w;
              o8[4] += p * v1.x;
              o8[5] += p * v1.y;
              o8[6] += p * v1.z;
              o8[7] += p * v1.w;
            } else {
              const uint4 vq = *reinterpret_cast<const uint4 *>(kvs + ((kKeyPasses + ps) * kLoadThreads + ll) * 4);
              const uint32_t w[4] = {vq.x, vq.y, vq.z, vq.w};
#pragma unroll
              for (int e = 0; e < 4; e++) {
                o8[2 * e] += p * __uint_as_float(w[e] << 16);
                o8[2 * e + 1] += p * __uint_as_float(w[e] & 0xffff0000u);
              }
            }
          }
        }
        lsum = wave64_sum(lsum);
        // lanes i and i+8 of a 16-lane row share a dimension slice: fold them (row_ror:8),
        // then the low half of every row writes its 8 dimensions; the K staging area is
        // free since the scores are done (the barrier above)
        float *ow2 = kvs;  // [9 waves][4 rows][64 dims]
#pragma unroll
        for (int e = 0; e < 8; e++) o8[e] += dpp_f<0x128, 0xf, 0xf>(o8[e], 0.0f);
        if ((lane & 15) < 8) {
          float *dst = ow2 + (lw * 4 + (lane >> 4)) * 64 + dsl * 8;
          *reinterpret_cast<float4 *>(dst) = make_float4(o8[0], o8[1], o8[2], o8[3]);
          *reinterpret_cast<float4 *>(dst + 4) = make_float4(o8[4], o8[5], o8[6], o8[7]);
        }
        if (lane == 0) sh.l_w[lw] = lsum;
      }
      __syncthreads();
      // block partial -> exchange (publisher); the split counter (a poller, which has no
      // stores in flight) names the last split of the head to finish, which combines
      if (pub) {
        float osum = 0.0f;
        for (int w = 0; w < kLoadWaves * 4; w++) osum += kvs[w * 64 + lane];
        float lt = 0.0f;
        for (int w = 0; w < kLoadWaves; w++) lt += sh.l_w[w];
        // [M, l, o0..o63] staged in qs (free after the scores) for the word layout
        qs[2 + lane] = osum;
        if (lane == 0) {
          qs[0] = M;
          qs[1] = lt;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane < kPartWords) {
          const int e0 = 3 * lane;
          xstore(x_part + (ah * S + aj) * kPartWords + lane, qs[e0], e0 + 1 < kPartVals ? qs[e0 + 1] : 0.0f,
                 e0 + 2 < kPartVals ? qs[e0 + 2] : 0.0f, ep + 2u);
        }
      }
      if (poller && T == 0) {
        // wrapping device-scope counter: cycles 0..S-1, so the S-th arrival reads S-1
        const uint32_t old = atomicInc(a.cnt + ah * kCntStride, (uint32_t)(S - 1));
        sh.last = old == (uint32_t)(S - 1);
      }
      __syncthreads();
      if (sh.last) {
        if (poller && !poll(
                          S * kPartWords, ep + 2u, err, T,
                          [&](int i) { return x_part + ah * S * kPartWords + i; },
                          [&](int i, u32x4 v) {
                            const int s = i / kPartWords;
                            put_word(pp + s * kPartVals, i - s * kPartWords, kPartVals, v);
                          }))
          sh.abort = 1;
        __syncthreads();
        if (sh.abort) return;
        if (pub) {
          float Mg = -INFINITY;
          for (int s = 0; s < S; s++) Mg = fmaxf(Mg, pp[s * kPartVals]);
          float den = 0.0f, num = 0.0f;
          for (int s = 0; s < S; s++) {
            if (pp[s * kPartVals] == -INFINITY) continue;
            const float f = __expf(pp[s * kPartVals] - Mg);
            den += pp[s * kPartVals + 1] * f;
            num += pp[s * kPartVals + 2 + lane] * f;
          }
          qs[lane] = num / den;  // staged for the word layout
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (lane < kHeadWords) {
            const int e0 = 3 * lane;
            xstore(x_attn + ah * kHeadWords + lane, qs[e0], e0 + 1 < 64 ? qs[e0 + 1] : 0.0f,
                   e0 + 2 < 64 ? qs[e0 + 2] : 0.0f, ep + 3u);
          }
        }
      }
    }
    // Weight prefetch: this layer's c_fc and mlp c_proj slices and the next layer's QKV
    // slice (18 MB across the chip), issued together once the attention is done.  A burst
    // of this size delays the exchange that follows it: ahead of the q/k/v, x_mid or x_f
    // exchange by 2-3 us each, ahead of the attention all-gather (whose split counter and
    // combine are latency-bound) far less; all three here measured 557 us per step against
    // 596 us with each issued after the phase before its own use.  The barrier puts the
    // publisher's exchange stores (the attention partial) ahead of the burst in the memory
    // pipeline (547 against 557 us).  The matrices' code pointers come from the layer
    // table by vector loads, which complete in issue order, so each matrix's loads start
    // once the previous matrix's have landed: the burst goes out in three waves.  Read
    // through the constant address space (scalar loads), the table let all three go out at
    // once, and the step took 546 against 526 us.
    __syncthreads();
    if (loader) load_slots<BITS, PT>(wf, Ly.fc, m_fc, ll);
    if (loader) load_slots<BITS, PT>(wm, Ly.mproj, m_mp, ll);
    if (loader && l + 1 < a.n_layer) load_slots<BITS, PT>(wq, a.layers[l + 1].attn, m_qkv, ll);
    // ---------------- P3: c_proj rows + residual ------------------------------------
    if (poller && !poll(
                      H * kHeadWords, ep + 3u, err, T, [&](int i) { return x_attn + i; },
                      [&](int i, u32x4 v) {
                        const int h = i / kHeadWords;
                        const int j = i - h * kHeadWords;
                        const float f[3] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z)};
#pragma unroll
                        for (int e = 0; e < 3; e++)
                          if (3 * j + e < 64) xin[xpad<BITS>(h * 64 + 3 * j + e)] = f[e];
                      }))
      sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    if (loader) dot_slots<BITS>(wp, m_proj, xin, part, ll);
    __syncthreads();
    if (loader)
      row_sums(m_proj, part, lw, lane, [&](int r, float v) {
        const float xm = own[r] + (v + lp[bo_p + r]);
        own_mid[r] = xm;
        out[r] = xm;
      });
    __syncthreads();
    if (pub) publish_rows(a.x_mid, d, B, b, out, m_proj.rows, ep + 4u, lane);
    // ---------------- P4: LN2, c_fc rows + GELU ------------------------------------
    if (poller && !poll_rows_ln<BITS>(a.x_mid, d, B, rs_d, ep + 4u, xin, xn, lp + d, err, T)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    if (poller) ln_stats(xin, d, sh.red, &sh.stat_cnt, T);
    if (loader) dot_slots<BITS>(wf, m_fc, xn, part, ll);
    __syncthreads();
    if (loader) {
      const float mu = sh.red[24], rstd = sh.red[25];
      row_sums(m_fc, part, lw, lane,
               [&](int r, float v) { out[r] = gelu_tanh_exp(rstd * (v - mu * lp[bo_gf + r]) + lp[bo_cf + r]); });
    }
    __syncthreads();
    if (pub) {
      publish_rows(a.x_f, F, B, b, out, m_fc.rows, ep + 5u, lane);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // next layer's parameter copies
    }
    // ---------------- P5: mlp c_proj rows + residual ---------------------------------
    if (poller && !poll_rows<BITS, true>(a.x_f, F, B, rs_f, ep + 5u, xin, err, T)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    if (loader) dot_slots<BITS>(wm, m_mp, xin, part, ll);
    __syncthreads();
    if (loader)
      row_sums(m_mp, part, lw, lane, [&](int r, float v) {
        const float xo = own_mid[r] + (v + lp[bo_m + r]);
        own[r] = xo;
        out[r] = xo;
      });
    __syncthreads();
    if (pub) publish_rows(a.x_x, d, B, b, out, m_mp.rows, ep + 6u, lane);
    __syncthreads();
  }
  // ---------------- head: ln_f, final_norm, mel_head rows -> logits ------------------
  {
    Slots<PT, kSlHead> wh;
    if (loader) load_slots<BITS, PT>(wh, a.head, m_head, ll);
    const uint32_t ep = ep0 + (uint32_t)(a.n_layer - 1) * 8u;
    const float *lp = lpb + (a.n_layer & 1) * a.lp_len;
    if (poller && !poll_rows<BITS, false>(a.x_x, d, B, rs_d, ep + 6u, xin, err, tid)) sh.abort = 1;
    __syncthreads();
    if (sh.abort) return;
    layer_norm(xin, xn, lp, lp + d, d, sh.red, tid);
    layer_norm(xn, xn, lp + 2 * d, lp + 3 * d, d, sh.red, tid, BITS == 8 ? 2 : 3);
    if (loader) dot_slots<BITS>(wh, m_head, xn, part, ll);
    __syncthreads();
    if (loader) row_sums(m_head, part, lw, lane, [&](int r, float v) { out[r] = v + lp[4 * d + r]; });
    __syncthreads();
    if (pub) {
      for (int r = lane; r < m_head.rows; r += 64) a.logits[m_head.row0 + r] = out[r];
      // Block 0 closes the step.  Every block read the control block at its start, before
      // its first exchange word, and block 0 gets here only after every block's last
      // exchange.
      if (b == 0 && lane == 0) {
        ctl->valid_len = vlen + 1;
        ctl->xstep = (int32_t)(xstep + 1u);
      }
    }
  }
}

template <int BITS, int PT, int KVF>
__global__ __launch_bounds__(kThreads) void decode_persist_kernel(PersistArgs a) {
  __shared__ PersistShared sh;
  // 16-byte aligned: the float4 LDS accesses assume it (the dynamic region follows sh)
  extern __shared__ __attribute__((aligned(16))) float lds[];
  if (a.ctl->done) return;
  if (threadIdx.x == 0) {
    sh.abort = 0;
    sh.last = 0;
    sh.stat_cnt = 0;
  }
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (wave >= kLoadWave0) {
    run<BITS, PT, KVF, kRoleLoad>(a, sh, lds);
  } else if (wave == kPubWave) {
    // the publisher's instructions issue ahead of the other waves' (the exchange stores,
    // which every block waits for, leave sooner): 524 against 535 us per step; raising
    // the pollers' priority as well changed nothing, raising theirs alone cost 5 us
    __builtin_amdgcn_s_setprio(3);
    run<BITS, PT, KVF, kRolePub>(a, sh, lds);
  } else {
    run<BITS, PT, KVF, kRolePoll>(a, sh, lds);
  }
}

template <int BITS, int PT>
const void *persist_fn_kv(int kvt) {
  return kvt == kKvF32 ? reinterpret_cast<const void *>(decode_persist_kernel<BITS, PT, 1>)
                       : reinterpret_cast<const void *>(decode_persist_kernel<BITS, PT, 0>);
}

const void *persist_fn(int bits, int ptype, int kvt) {
  if (bits == 4)
    return ptype == kParamF16 ? persist_fn_kv<4, kParamF16>(kvt) : persist_fn_kv<4, kParamF32>(kvt);
  return ptype == kParamF16 ? persist_fn_kv<8, kParamF16>(kvt) : persist_fn_kv<8, kParamF32>(kvt);
}

}  // namespace

namespace {

// One wave per row o of ql: G[o] = sum_k Wdeq[o][k] gamma[k], c[o] = sum_k Wdeq[o][k]
// beta[k] + bias[o], with Wdeq = s * q + b of the row's 64-groups (gpt.rs:221-264), summed in
// fp64 and rounded once.  Lane i takes columns i, i + 64, ... .
template <int BITS, int PT>
__global__ __launch_bounds__(256) void ln_fold_kernel(DevQL ql, const float *gamma, const float *beta, float *G,
                                                      float *c) {
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= ql.N) return;
  const int K = ql.K, ng = K / kGroup;
  double g_acc = 0.0, b_acc = 0.0;
  for (int g = 0; g < ng; g++) {
    float s, bb;
    if constexpr (PT == kParamF16) {
      const uint32_t w = static_cast<const uint32_t *>(ql.params)[(size_t)o * ng + g];
      s = half_bits_to_float(w & 0xffffu);
      bb = half_bits_to_float(w >> 16);
    } else {
      const float2 w = static_cast<const float2 *>(ql.params)[(size_t)o * ng + g];
      s = w.x;
      bb = w.y;
    }
    const int k = g * kGroup + lane;
    uint32_t q;
    if constexpr (BITS == 8)
      q = ql.codes[(size_t)o * K + k];
    else
      q = (ql.codes[((size_t)o * K + k) >> 1] >> (4 * (k & 1))) & 0xfu;
    const double w = (double)s * (double)q + (double)bb;
    g_acc += w * (double)gamma[k];
    b_acc += w * (double)beta[k];
  }
  for (int m = 32; m >= 1; m >>= 1) {
    g_acc += __shfl_xor(g_acc, m);
    b_acc += __shfl_xor(b_acc, m);
  }
  if (lane == 0) {
    G[o] = (float)g_acc;
    c[o] = (float)(b_acc + (double)ql.bias[o]);
  }
}

}  // namespace

hipError_t launch_ln_fold(const DevQL &ql, int bits, int ptype, const float *gamma, const float *beta, float *G,
                          float *c, hipStream_t s) {
  const dim3 grid((ql.N + 3) / 4), block(256);
  if (bits == 4) {
    if (ptype == kParamF16)
      ln_fold_kernel<4, kParamF16><<<grid, block, 0, s>>>(ql, gamma, beta, G, c);
    else
      ln_fold_kernel<4, kParamF32><<<grid, block, 0, s>>>(ql, gamma, beta, G, c);
  } else {
    if (ptype == kParamF16)
      ln_fold_kernel<8, kParamF16><<<grid, block, 0, s>>>(ql, gamma, beta, G, c);
    else
      ln_fold_kernel<8, kParamF32><<<grid, block, 0, s>>>(ql, gamma, beta, G, c);
  }
  return hipGetLastError();
}

bool persist_supported(int d, int F, int V, int H, int n_layer, int max_seq, int B, int bits, int *S_out) {
  // d <= 4 * kPollThreads: the folded LayerNorms' statistics take one float4 per poller lane
  if (B < 1 || H < 1 || d % 64 != 0 || d > 4 * kPollThreads || F % 64 != 0 || n_layer < 1 ||
      (bits != 8 && bits != 4))
    return false;
  const int epc = bits == 8 ? 16 : 32;
  const int S = std::min(12, B / H);
  if (S < 1) return false;
  if ((max_seq + S - 1) / S > kKeySlots * kKeyPasses) return false;
  // one publisher wave writes a block's words of any array
  if ((3 * d + B - 1) / B > 3 * 64 || (F + B - 1) / B > 3 * 64) return false;
  auto fits = [&](int N, int C, int slots) {
    return (long)((N + B - 1) / B) * C <= (long)slots * kLoadThreads;
  };
  if (!fits(3 * d, d / epc, kSlQkv) || !fits(d, d / epc, kSlProj) || !fits(F, d / epc, kSlFc) ||
      !fits(d, F / epc, kSlMp) || !fits(V, d / epc, kSlHead))
    return false;
  *S_out = S;
  return true;
}

size_t persist_exchange_words(int d, int F, int H, int S, int B, size_t off[6]) {
  auto w = [&](int N) { return (size_t)B * (((N + B - 1) / B + 2) / 3); };
  const size_t n[6] = {w(d), w(3 * d), (size_t)H * S * kPartWords, (size_t)H * kHeadWords, w(d), w(F)};
  size_t t = 0;
  for (int i = 0; i < 6; i++) {
    off[i] = t;
    t += n[i];
  }
  return t;
}

size_t persist_lds_bytes(const PersistArgs &a) {
  const size_t f = (size_t)a.xin_len + a.xn_len + a.part_len + 2 * (size_t)a.own_len + a.out_len + 3 * 64 + a.pp_len +
                   2 * (size_t)a.lp_len + 2 * kKeyPasses * kLoadThreads * 4 + 3 * (size_t)(a.B + 1);
  return f * sizeof(float);
}

// A regular launch (a cooperative one costs ~17 us more per step on MI355X).  The blocks are
// co-resident without the cooperative guarantee: the grid is one block per CU, the block's
// LDS admits only one per CU (persist_fits), and the decoder's stream orders the launch after
// every earlier kernel of the decoder.  Should another stream's work hold a CU anyway, the
// resident blocks' polls time out (bounded waits) and the step returns an error instead of
// waiting forever.
hipError_t launch_decode_persist(PersistArgs a, int bits, int ptype, hipStream_t s) {
  void *args[] = {&a};
  const size_t lds = persist_lds_bytes(a);
  return hipLaunchKernel(persist_fn(bits, ptype, a.kvt), dim3(a.B), dim3(kThreads), args, lds, s);
}

hipError_t persist_init() {
  for (int bits : {8, 4})
    for (int pt : {kParamF16, kParamF32})
      for (int kvt : {kKvBf16, kKvF32}) {
        hipError_t e = hipFuncSetAttribute(persist_fn(bits, pt, kvt), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)kPersistMaxLds);
        if (e != hipSuccess) return e;
      }
  return hipSuccess;
}

hipError_t persist_fits(int bits, int ptype, int kvt, size_t lds, bool *fits) {
  const void *fn = persist_fn(bits, ptype, kvt);
  hipFuncAttributes fa{};
  hipError_t e = hipFuncGetAttributes(&fa, fn);
  if (e != hipSuccess) return e;
  int dev = 0, max_lds = 0;
  if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
  if ((e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev)) != hipSuccess)
    return e;
  // 1024 threads use the whole CU (16 waves); the compiler bounded the registers for that
  // (launch bounds), so the block fits when its LDS does
  *fits = fa.maxThreadsPerBlock >= kThreads && fa.sharedSizeBytes + lds <= (size_t)max_lds &&
          lds <= kPersistMaxLds;
  return hipSuccess;
}

}  // namespace itts
