// sample_next_token (sampler.rs:191-284) as one 1024-thread block's device function, used by
// the sampler kernel (one block per sequence: single decode, batched decode, and the
// standalone itts_sample_next_token call).
//
// Bit-exactness.  Given the same fp32 logits, this returns the token the reference's
// algorithm returns: every value-producing operation is the same IEEE operation in the
// same order (penalty multiply/divide, x * (1/T), the exponential below, the sequential
// fp32 sums over the sorted candidates, the SplitMix64 draw).  Only the top-k selection
// and sorting are parallel, and they are order-exact: the candidates are ranked by
// (value desc, index asc) — the total order that pins down the reference's unstable sort
// on ties.
//
// Stages: (1) each thread holds up to 9 consecutive logits in registers, applies the
// STOP mask and the repetition penalty; (2) greedy: block argmax; (3) otherwise scale by
// 1/T, radix-select the k-th largest key (4 passes of 8 bits over an order-preserving
// 32-bit key; the first pass, which counts every key into few bins, spreads its LDS
// atomics over 16 padded histogram copies), take ties at the threshold by lowest index
// (block prefix scan), sort the k candidates (one wave in registers for k <= 64, else a
// block-wide bitonic network in LDS); (4) the probabilities' sequential prefix sums, the
// top-p cut and the draw: for k <= 64 by the sorting wave in registers (uniform loops of
// single adds over values read lane by lane), else by one thread over LDS.
#pragma once

#include "common.h"

namespace itts {

constexpr int kSampThreads = 1024;
constexpr int kSampPerThread = 9;  // n <= 9216
constexpr int kHistCopies = 16, kHistStride = 257;  // radix pass 0's histogram copies

// Every multiply and add below rounds on its own (no FMA contraction), as the reference's
// scalar Rust code does; the exponential uses explicit fmaf where intended.

// exp by Cody-Waite reduction with ln2 split and a degree-7 Taylor polynomial in
// Horner form; results below FLT_MIN flush to +0.
__device__ inline float sampler_expf(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -87.33654022216797f) return 0.0f;
  const float n = __builtin_rintf(mul_rn(x, 1.44269502162933349609375f));
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float y = ldexpf(p, (int)n);
  return y < 1.17549435082228751e-38f ? 0.0f : y;
}

__device__ inline uint64_t splitmix_next(uint64_t *state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ inline bool is_finite(float v) { return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u; }

// Order-preserving key of a non-NaN float, with -0 == +0.
__device__ inline uint32_t order_key(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline float key_value(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

struct SamplerShared {  // the sampler's LDS scratch (besides the sort keys)
  uint32_t hist[kHistCopies * kHistStride];
  int32_t wave_tot[kSampThreads / 64];
  int32_t scal[8];
  float fred[kSampThreads / 64];
  int32_t ired[kSampThreads / 64];
};


__device__ __forceinline__ float lane_f(float v, int i) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// Stage (4) for k <= 64 candidates held by one wave, sorted (lane i: candidate i, key
// (order key << 32 | ~id), lanes >= k zero): p_i = exp(v_i - v_0), the sequential fp32
// sums S_i = p_0 + .. + p_i (left to right, one add at a time, as the reference's loops
// run), the top-p cut over the normalised p_i / S_{k-1} (cumulated in the same order), and
// the draw u * S_{active-1} against S_0, S_1, ..  Each loop over i is a uniform loop of
// single adds on values read from lane i, so every sum is the serial one, bit for bit.
__device__ inline int32_t sample_sorted_wave(uint64_t x, int k, const DevSampling &p, uint64_t *rng) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const uint32_t kx = (uint32_t)(x >> 32);
  const int32_t id = (int32_t)(0xffffffffu - (uint32_t)x);
  const float v0 = key_value((uint32_t)__builtin_amdgcn_readlane((int)kx, 0));
  const float mx = is_finite(v0) ? v0 : 0.0f;
  const float vi = key_value(kx);
  const float pi = lane < k && is_finite(vi) ? sampler_expf(sub_rn(vi, mx)) : 0.0f;
  float s = 0.0f, S = 0.0f;
  for (int i = 0; i < k; i++) {
    s = add_rn(s, lane_f(pi, i));
    if (lane == i) S = s;
  }
  const float prob_sum = s;
  int32_t tok = __builtin_amdgcn_readlane(id, 0);
  if (prob_sum > 0.0f && is_finite(prob_sum)) {
    const float norm = div_rn(pi, prob_sum);
    float cum = 0.0f;
    int active = k;
    for (int i = 0; i < k; i++) {
      if (i > 0 && cum > p.top_p) {
        active = i;
        break;
      }
      cum = add_rn(cum, lane_f(norm, i));
    }
    const float active_sum = lane_f(S, active - 1);
    if (active_sum > 0.0f && is_finite(active_sum)) {
      uint32_t upper = 0;
      if (lane == 0) upper = (uint32_t)(splitmix_next(rng) >> 40);
      upper = (uint32_t)__builtin_amdgcn_readlane((int)upper, 0);
      const float u = mul_rn((float)upper, 1.0f / 16777216.0f);
      const float draw = mul_rn(u, active_sum);
      const uint64_t hit = __ballot(lane < active && draw <= S);
      tok = __builtin_amdgcn_readlane(id, hit ? (int)__builtin_ctzll(hit) : active - 1);
    }
  }
  return tok;
}

// The token sample_next_token returns for logits src[0..n) (read only; LDS or global), run
// by all kSampThreads threads of the block, which all get the result.  seen: the penalty
// set; *rng: the SamplerRng state, advanced by thread 0 on a draw; mask_stop: logit
// stop_tok is -inf (generate_codes_after's min_codes rule); penalised_out (optional):
// receives the penalised logits; sk: LDS sort keys, next_pow2(p.top_k) entries.
__device__ __forceinline__ int32_t sample_block(const float *src, float *penalised_out, int n, const uint64_t *seen,
                                                const DevSampling &p, uint64_t *rng, bool mask_stop, int stop_tok,
                                                SamplerShared &sh, uint64_t *sk) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = (n + kSampThreads - 1) / kSampThreads;
  const int i0 = tid * E;
  // (1) load, STOP mask, repetition penalty (x<0 ? x*p : x/p).  Every load is issued before
  // the first store (penalised_out may be src), and the thread's E <= 9 consecutive ids
  // span at most two seen words, read once.
  float v[kSampPerThread];
#pragma unroll
  for (int e = 0; e < kSampPerThread; e++) v[e] = e < E && i0 + e < n ? src[i0 + e] : 0.0f;
  const int w0 = i0 >> 6;
  const uint64_t sw0 = p.apply_penalty && w0 < kSeenWords ? seen[w0] : 0ull;
  const uint64_t sw1 = p.apply_penalty && w0 + 1 < kSeenWords ? seen[w0 + 1] : 0ull;
#pragma unroll
  for (int e = 0; e < kSampPerThread; e++) {
    const int i = i0 + e;
    if (e < E && i < n) {
      float x = v[e];
      if (mask_stop && i == stop_tok) x = -INFINITY;
      const uint64_t sw = (i >> 6) == w0 ? sw0 : sw1;
      if (p.apply_penalty && (i >> 6) < kSeenWords && ((sw >> (i & 63)) & 1ull)) {
        x = x < 0.0f ? mul_rn(x, p.penalty) : div_rn(x, p.penalty);
      }
      v[e] = x;
    }
  }
  if (penalised_out) {
#pragma unroll
    for (int e = 0; e < kSampPerThread; e++)
      if (e < E && i0 + e < n) penalised_out[i0 + e] = v[e];
  }

  int32_t result = 0;
  if (p.greedy) {
    // (2) first index of the strict maximum over finite values; 0 if none is finite.
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < kSampPerThread; e++) {
      const int i = i0 + e;
      if (e < E && i < n && is_finite(v[e]) && v[e] > bv) {
        bv = v[e];
        bi = i;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      sh.fred[wave] = bv;
      sh.ired[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      float gv = -INFINITY;
      int gi = 0x7fffffff;
      for (int w = 0; w < kSampThreads / 64; w++) {
        if (sh.fred[w] > gv || (sh.fred[w] == gv && sh.ired[w] < gi)) {
          gv = sh.fred[w];
          gi = sh.ired[w];
        }
      }
      sh.scal[0] = gi == 0x7fffffff ? 0 : gi;
    }
    __syncthreads();
    result = sh.scal[0];
  } else {
    // (3) temperature, then keys
    uint32_t key[kSampPerThread];
#pragma unroll
    for (int e = 0; e < kSampPerThread; e++) {
      const int i = i0 + e;
      const bool live = e < E && i < n;
      const float s = is_finite(v[e]) ? mul_rn(v[e], p.inv_temp) : -INFINITY;
      v[e] = s;
      key[e] = live ? order_key(s) : 0u;  // padding sorts below -inf (key 0x007fffff)
    }
    const int k = p.top_k;
    // radix select of the k-th largest key
    uint32_t prefix = 0, pmask = 0;
    int remaining = k;
    for (int pass = 0; pass < 4; pass++) {
      const int shift = 24 - 8 * pass;
      // pass 0 counts every key, whose top byte (sign and exponent) takes few values: the
      // counts go to kHistCopies copies (by lane), padded apart so that lanes with one bin
      // hit distinct LDS banks; later passes count few keys, into copy 0
      const int copies = pass == 0 ? kHistCopies : 1;
      for (int b = tid; b < copies * kHistStride; b += kSampThreads) sh.hist[b] = 0;
      __syncthreads();
      uint32_t *hcopy = sh.hist + (pass == 0 ? (lane % kHistCopies) * kHistStride : 0);
#pragma unroll
      for (int e = 0; e < kSampPerThread; e++) {
        const int i = i0 + e;
        if (e < E && i < n && (key[e] & pmask) == prefix) atomicAdd(&hcopy[(key[e] >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (wave == 0) {
        // lane l covers bins 255-4l .. 252-4l (descending)
        uint32_t c[4];
        uint32_t tot = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          c[j] = 0;
          for (int cp = 0; cp < copies; cp++) c[j] += sh.hist[cp * kHistStride + 255 - 4 * lane - j];
          tot += c[j];
        }
        uint32_t incl = tot;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t o = __shfl_up(incl, off, 64);
          if (lane >= off) incl += o;
        }
        uint32_t above = incl - tot;  // elements in strictly higher bins
        if (above < (uint32_t)remaining && (uint32_t)remaining <= incl) {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            if (above < (uint32_t)remaining && (uint32_t)remaining <= above + c[j]) {
              sh.scal[0] = 255 - 4 * lane - j;
              sh.scal[1] = (int)above;
            }
            above += c[j];
          }
        }
      }
      __syncthreads();
      const uint32_t digit = (uint32_t)sh.scal[0];
      remaining -= sh.scal[1];
      prefix |= digit << shift;
      pmask |= 0xffu << shift;
      __syncthreads();
    }
    const uint32_t thr = prefix;  // key of the k-th largest; `remaining` ties to take
    // ties at the threshold: take the `remaining` lowest indices (prefix scan in index order)
    int my_eq = 0;
#pragma unroll
    for (int e = 0; e < kSampPerThread; e++) {
      const int i = i0 + e;
      if (e < E && i < n && key[e] == thr) my_eq++;
    }
    int incl = my_eq;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    if (lane == 63) sh.wave_tot[wave] = incl;
    if (tid == 0) sh.scal[2] = 0;  // candidate counter
    __syncthreads();
    int eq_before = incl - my_eq;
    for (int w = 0; w < wave; w++) eq_before += sh.wave_tot[w];
    const int P = (int)next_pow2((uint32_t)k);
#pragma unroll
    for (int e = 0; e < kSampPerThread; e++) {
      const int i = i0 + e;
      if (!(e < E && i < n)) continue;
      bool take = key[e] > thr;
      if (key[e] == thr) {
        take = eq_before < remaining;
        eq_before++;
      }
      if (take) {
        const int slot = atomicAdd(&sh.scal[2], 1);
        if (slot < k) sk[slot] = ((uint64_t)key[e] << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
      }
    }
    __syncthreads();
    if (P <= 64) {
      // one wave sorts the candidates in registers (bitonic network over lane pairs, descending;
      // keys are distinct, so the order equals the block-wide network's), then forms the
      // probabilities, their sequential sums, the top-p cut and the draw in registers
      if (wave == 0) {
        uint64_t x = lane < k ? sk[lane] : 0ull;
        for (int size = 2; size <= 64; size <<= 1)
          for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t ylo = (uint32_t)__shfl_xor((int)(uint32_t)x, stride, 64);
            const uint32_t yhi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), stride, 64);
            const uint64_t y = ((uint64_t)yhi << 32) | ylo;
            const bool keep_max = ((lane & size) == 0) == ((lane & stride) == 0);
            x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
          }
        const int32_t tok = sample_sorted_wave(x, k, p, rng);
        if (lane == 0) sh.scal[3] = tok;
      }
      __syncthreads();
      return sh.scal[3];
    }
    for (int i = k + tid; i < P; i += kSampThreads) sk[i] = 0ull;
    __syncthreads();
    // bitonic sort, descending
    for (int size = 2; size <= P; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < P / 2; t += kSampThreads) {
          const int i = 2 * t - (t & (stride - 1));
          const int j = i + stride;
          const bool desc = (i & size) == 0;
          const uint64_t x = sk[i], y = sk[j];
          if ((x < y) == desc) {
            sk[i] = y;
            sk[j] = x;
          }
        }
        __syncthreads();
      }
    }
    // (4) probabilities p_i = exp(v_i - max); repack as (p bits << 32 | id)
    const float v0 = key_value((uint32_t)(sk[0] >> 32));
    const float mx = is_finite(v0) ? v0 : 0.0f;
    for (int i = tid; i < k; i += kSampThreads) {
      const uint64_t e = sk[i];
      const float vi = key_value((uint32_t)(e >> 32));
      const uint32_t id = 0xffffffffu - (uint32_t)e;
      const float pi = is_finite(vi) ? sampler_expf(sub_rn(vi, mx)) : 0.0f;
      sk[i] = ((uint64_t)__float_as_uint(pi) << 32) | id;
    }
    __syncthreads();
    if (tid == 0) {
      float prob_sum = 0.0f;
      for (int i = 0; i < k; i++) prob_sum = add_rn(prob_sum, __uint_as_float((uint32_t)(sk[i] >> 32)));
      int32_t tok = (int32_t)(uint32_t)sk[0];
      if (prob_sum > 0.0f && is_finite(prob_sum)) {
        float cum = 0.0f;
        int active = k;
        for (int i = 0; i < k; i++) {
          const float norm = div_rn(__uint_as_float((uint32_t)(sk[i] >> 32)), prob_sum);
          if (i > 0 && cum > p.top_p) {
            active = i;
            break;
          }
          cum = add_rn(cum, norm);
        }
        float active_sum = 0.0f;
        for (int i = 0; i < active; i++) active_sum = add_rn(active_sum, __uint_as_float((uint32_t)(sk[i] >> 32)));
        if (active_sum > 0.0f && is_finite(active_sum)) {
          const uint32_t upper = (uint32_t)(splitmix_next(rng) >> 40);
          const float u = mul_rn((float)upper, 1.0f / 16777216.0f);
          const float draw = mul_rn(u, active_sum);
          float accp = 0.0f;
          tok = (int32_t)(uint32_t)sk[active - 1];
          for (int i = 0; i < active; i++) {
            accp = add_rn(accp, __uint_as_float((uint32_t)(sk[i] >> 32)));
            if (draw <= accp) {
              tok = (int32_t)(uint32_t)sk[i];
              break;
            }
          }
        }
      }
      sh.scal[3] = tok;
    }
    __syncthreads();
    result = sh.scal[3];
  }

  return result;
}

// generate_codes_after's bookkeeping after sample s (sampler.rs:378-388): STOP ends the
// generation; otherwise the code is emitted, marked seen, and becomes the next step's token
// at position n_prior + s + 2 unless s was the last step.  Thread 0 only.  Every field is
// read before the first store: read between the stores (which the compiler cannot prove
// apart from them), each read would wait for the stores before it.
__device__ inline void sampler_commit(DecodeCtl *c, uint64_t *seen, int32_t result, int stop_tok, int32_t *codes) {
  const int n_codes = c->n_codes, s = c->step, max_steps = c->max_steps, n_prior = c->n_prior;
  const bool stop = result == stop_tok, mark = !stop && result >= 0 && result < kSeenWords * 64;
  const uint64_t word = mark ? seen[result >> 6] : 0ull;
  c->last_tok = result;
  if (stop) {
    c->done = 1;
  } else {
    codes[n_codes] = result;
    c->n_codes = n_codes + 1;
    if (mark) seen[result >> 6] = word | (1ull << (result & 63));
    if (s + 1 < max_steps) {
      c->tok = result;
      c->pos = n_prior + s + 2;
    } else {
      c->done = 1;
    }
  }
  c->step = s + 1;
}

}  // namespace itts
