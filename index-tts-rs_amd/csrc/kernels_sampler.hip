// On-device sampler: sample_next_token (sampler.rs:191-284) in one 1024-thread block; the
// algorithm and its bit-exactness argument are in sampler_core.h.
#include "kernels.h"
#include "sampler_core.h"

namespace itts {

namespace {

constexpr int kThreads = kSampThreads;
constexpr int kPerThread = kSampPerThread;

// mode 0: API call on `logits` (penalised in place, token to *tok_out, rng advanced);
// mode 1: generate step driven by ctl (seen, rng, min_codes, bookkeeping); batch mode
// (seqs != nullptr): block b serves sequence b with its own logits row, ctl and params.
__global__ __launch_bounds__(kThreads) void sampler_kernel(float *logits, int n, const uint64_t *seen_in,
                                                           DevSampling p, uint64_t *rng_in,
                                                           int32_t *tok_out, DecodeCtl *ctl,
                                                           int32_t *codes, int stop_tok, int mode,
                                                           const DevSampling *ps, const BatchSeq *seqs) {
  __shared__ SamplerShared sh;
  extern __shared__ uint64_t sk[];  // [P] sort keys
  if (seqs != nullptr) {
    ctl = seqs[blockIdx.x].ctl;
    codes = seqs[blockIdx.x].codes;
    p = ps[blockIdx.x];
    logits += (size_t)blockIdx.x * n;
  }
  if (mode == 1 && ctl->done) return;
  const uint64_t *seen = mode == 1 ? ctl->seen : seen_in;
  uint64_t *rng = mode == 1 ? &ctl->rng : rng_in;
  const bool mask_stop = mode == 1 && ctl->n_codes < ctl->min_codes;
  const int32_t result = sample_block(logits, mode == 0 ? logits : nullptr, n, seen, p, rng, mask_stop, stop_tok, sh, sk);
  if (threadIdx.x == 0) {
    if (mode == 0)
      *tok_out = result;
    else
      sampler_commit(ctl, ctl->seen, result, stop_tok, codes);
  }
}

}  // namespace

hipError_t sampler_init() {
  // candidate sort keys for top_k up to 8194 need 128 KiB of LDS
  return hipFuncSetAttribute(reinterpret_cast<const void *>(sampler_kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, 131072);
}

hipError_t launch_sampler(float *logits, int n, const uint64_t *seen, DevSampling p,
                          uint64_t *rng, int32_t *tok_out, DecodeCtl *ctl, int32_t *codes,
                          int stop_tok, int mode, hipStream_t s) {
  if (n <= 0 || n > kThreads * kPerThread) return hipErrorInvalidValue;
  size_t lds = 8;
  if (!p.greedy) {
    if (p.top_k < 1 || p.top_k > n) return hipErrorInvalidValue;
    lds = sizeof(uint64_t) * next_pow2((uint32_t)p.top_k);
  }
  hipLaunchKernelGGL(sampler_kernel, dim3(1), dim3(kThreads), lds, s, logits, n, seen, p, rng,
                     tok_out, ctl, codes, stop_tok, mode, nullptr, nullptr);
  return hipGetLastError();
}

hipError_t launch_sampler_batch(float *logits, int n, const DevSampling *ps, const BatchSeq *seqs, int B,
                                int stop_tok, int lds_top_k, bool any_sampled, hipStream_t s) {
  if (n <= 0 || n > kThreads * kPerThread || B <= 0) return hipErrorInvalidValue;
  size_t lds = 8;
  if (any_sampled) {
    if (lds_top_k < 1 || lds_top_k > n) return hipErrorInvalidValue;
    lds = sizeof(uint64_t) * next_pow2((uint32_t)lds_top_k);
  }
  hipLaunchKernelGGL(sampler_kernel, dim3(B), dim3(kThreads), lds, s, logits, n, nullptr, DevSampling{}, nullptr,
                     nullptr, nullptr, nullptr, stop_tok, 1, ps, seqs);
  return hipGetLastError();
}

}  // namespace itts
