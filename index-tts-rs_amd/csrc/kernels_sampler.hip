// On-device sampler: sample_next_token (sampler.rs:191-284) in one 1024-thread block; the
// algorithm and its bit-exactness argument are in sampler_core.h.
#include <mutex>

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

// ---- staging without allocation ----------------------------------------------------
// Byte offsets inside the staging array: logits, seen words, RNG state, token.
constexpr size_t kStageSeenOff = sizeof(float) * kStageMaxLogits;
constexpr size_t kStageRngOff = kStageSeenOff + sizeof(uint64_t) * 129;
constexpr size_t kStageTokOff = kStageRngOff + sizeof(uint64_t);
constexpr size_t kStageBytes = (kStageTokOff + sizeof(int32_t) + 255) / 256 * 256;  // 38144
static_assert(kStageMaxLogits <= kThreads * kPerThread, "the sampler block must cover the staging area");

// In host code `scratch` names a host-side stand-in, not device memory: host code uses the
// address hipGetSymbolAddress returns for each device (g_stage_dev), never the name.
static __device__ __align__(256) unsigned char scratch[kStageBytes];

std::mutex g_stage_mu;
char *g_stage_dev[kMaxDevices];  // per-device address of `scratch`

}  // namespace

hipError_t sampler_stage_init(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_stage_mu);
  if (g_stage_dev[dev]) return hipSuccess;
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!ptr) return hipErrorInvalidSymbol;
  g_stage_dev[dev] = static_cast<char *>(ptr);
  return hipSuccess;
}

bool sampler_stage(int dev, SamplerStage *out) {
  if (dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_stage_mu);
  char *base = g_stage_dev[dev];
  if (!base) return false;
  out->logits = reinterpret_cast<float *>(base);
  out->seen = reinterpret_cast<uint64_t *>(base + kStageSeenOff);
  out->rng = reinterpret_cast<uint64_t *>(base + kStageRngOff);
  out->tok = reinterpret_cast<int32_t *>(base + kStageTokOff);
  return true;
}

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
