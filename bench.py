"""Benchmark of the int8 GPT-2 semantic-token decoder on one MI355X.

Workload (default): the long-utterance configuration — 24 layers, d_model 1280,
20 heads, int8 group-64 weights with fp16 group params (seeded N(0, 0.02) init),
batch 1, prefill 32 conditioning rows + 200 text tokens (235 rows), then 1500 sampled
decode steps (temperature 0.8, top-k 30, top-p 0.8, repetition penalty 10, fixed seed,
STOP masked so the length is fixed), bf16 KV cache growing to 1734 rows.

One benchmark step = one whole generation (prefill + 1500 sampled tokens) through
itts_generate_codes_after, inputs already resident on the device.  `value` is generated
tokens per second over the timed steps (prefill included).  The decode step (one
replay of the captured sample+step graph) is the unit whose HBM roofline is reported:
achieved = algorithmic bytes of one decode step / its average device time (HIP events
on the decoder's stream).

The default run also reports, under "secondary", the short workload, the long workload
with an fp32 cache, the prefill-heavy workload (4 x 547 rows, all-row logits,
MFMA-bound), the batch-8 decode workload, the int4 decode workload and the Stage-2 CFM
estimator's 25-step solve for 10 s of audio.

Usage: python bench.py [--steps K] [--warmup W] [--workload long|short|int4]
"""
import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "index-tts-rs_amd"))

import numpy as np  # noqa: E402

METRIC = "batch-1 decode tokens/s (int8, 24L d1280); % of HBM roofline; TTFT"
HBM_PEAK_GBS = 8000.0
KV_ROW_BYTES = 24 * 2 * 20 * 64 * 2  # one position of K and V over 24 layers, bf16

WORKLOADS = {
    # name: (n_cond, n_text, steps, sampling, bits, description)
    "long": (32, 200, 1500, dict(greedy=False, temperature=0.8, top_k=30, top_p=0.8,
                                  repetition_penalty=10.0),
             8, "batch 1, prefill 32 cond + 200 text (235 rows), 1500 sampled steps "
                "(T 0.8, top-k 30, top-p 0.8, penalty 10), bf16 KV to 1734 rows"),
    "short": (32, 64, 128, dict(greedy=True, repetition_penalty=10.0), 8,
              "batch 1, prefill 32 cond + 64 text (99 rows), 128 greedy steps"),
    "int4": (32, 128, 1500, dict(greedy=True, repetition_penalty=10.0), 4,
             "int4 weights, batch 1, prefill 32 + 128 text (163 rows), 1500 greedy steps"),
}


def hip():
    lib = C.CDLL("libamdhip64.so")
    lib.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    lib.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    lib.hipEventSynchronize.argtypes = [C.c_void_p]
    lib.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    lib.hipDeviceSynchronize.argtypes = []
    return lib


def step_bytes(weight_bytes: int, L: int) -> int:
    """Algorithmic HBM bytes of one decode step with L keys (the new row included):
    every weight byte once, the K/V rows 0..L-1 once, the new K/V row written, the
    logits written."""
    return weight_bytes + KV_ROW_BYTES * L + KV_ROW_BYTES + 8194 * 4


MFMA_PEAK_TFLOPS = 2500.0  # fp16 dense, MI355X


def prefill_flops(T: int, d=1280, F=5120, V=8194, layers=24, heads=20, hd=64) -> float:
    """Algorithmic FLOPs of a T-row prefill (gpt.rs:636-696): the four linears of every
    block over all rows, causal attention (QK^T and PV over the T(T+1)/2 visible pairs
    of each head), and mel_head on the last row only."""
    lin = 2.0 * T * layers * (d * 3 * d + d * d + d * F + F * d)
    att = 2.0 * 2.0 * layers * heads * hd * (T * (T + 1) / 2)
    return lin + att + 2.0 * d * V


def ttft_roofline(ttft_ms: float, prefill_ms: float, T: int, weight_bytes: int) -> dict:
    """Time to first token against its roofline: the prefill's algorithmic FLOPs at the
    fp16 dense MFMA peak and its algorithmic bytes (every weight once, the T K/V rows
    written, the logits) at the HBM peak; the bound is the larger of the two times."""
    flop = prefill_flops(T)
    nbytes = weight_bytes + KV_ROW_BYTES * T + 8194 * 4
    t_mfma = flop / (MFMA_PEAK_TFLOPS * 1e12) * 1e3
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9) * 1e3
    bound_ms = max(t_mfma, t_hbm)
    return {"ttft_ms": round(ttft_ms, 3), "prefill_device_ms": round(prefill_ms, 3), "rows": T,
            "flop": round(flop), "bytes": nbytes,
            "bound": "mfma" if t_mfma >= t_hbm else "hbm",
            "roofline_ms": round(bound_ms, 4),
            "achieved_tflops": round(flop / (ttft_ms * 1e-3) / 1e12, 1),
            "frac": round(bound_ms / ttft_ms, 4),
            "frac_prefill_device": round(bound_ms / prefill_ms, 4),
            "note": "frac = roofline time / time; ttft is host call to the first token id on the host "
                    "(prefill + one sample), prefill_device_ms the prefill's HIP-event time"}


def cpu_baseline(W, prompt, sp, n_steps: int, prior):
    """The oracle (CPU restatement of the reference decoder) on the same weights: the
    prompt's prefill (CPU time to first token), then, from a cache holding the prompt and
    `prior` (the GPU run's first codes, so the context is the workload's mean), n_steps
    sampled decode steps; threads = host cores (<= 16)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ito

    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    ito.lib.ito_set_threads(threads)
    M = ito.Model(W)
    t0 = time.perf_counter()
    M.prefill_after(M.kv(2048, kv_bf16=True), prompt.text_tokens, prompt.conds, prompt.lang_id)
    t_prefill = time.perf_counter() - t0
    kv = M.kv(2048, kv_bf16=True)
    prior = np.ascontiguousarray(prior, np.int32)
    logits = M.prefill_after(kv, prompt.text_tokens, prompt.conds, prompt.lang_id, prior)
    L0 = kv.valid_len()
    seen = ito.seen_init()
    for t in prior.tolist():
        ito.lib.ito_seen_insert(ito._p(seen), int(t))
    state = ito.lib.ito_rng_init(1234)
    t0 = time.perf_counter()
    for s in range(n_steps):
        logits[8193] = -np.inf
        tok, state = ito.sample_next_token(logits, seen, sp, state)
        ito.lib.ito_seen_insert(ito._p(seen), tok)
        logits = M.step(kv, tok, len(prior) + s + 2)
    t_dec = time.perf_counter() - t0
    return {
        "value": round(n_steps / t_dec, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle (C restatement of gpt.rs/sampler.rs, fp32, bf16 KV) on the same weights: "
                  f"{n_steps} sampled decode steps at {L0 + 1}..{L0 + n_steps} keys (the GPU "
                  f"workload's mean context, after prefilling the prompt and the GPU run's first "
                  f"{len(prior)} codes), {t_dec * 1e3 / n_steps:.1f} ms/token; the {L0 - len(prior)}-row "
                  f"prompt prefill (CPU time to first token) took {t_prefill * 1e3:.0f} ms",
        "ttft_ms": round(t_prefill * 1e3, 1),
    }


def source_hash() -> str:
    """sha256 of the persistent step kernel's source (the GPU box has no git metadata)."""
    import hashlib
    with open(os.path.join(ROOT, "index-tts-rs_amd", "csrc", "kernels_persist.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_traffic(decode_path):
    """HBM bytes per launch of the persistent step from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), with whether it was
    measured on the kernel source built here; None if there is no summary."""
    if decode_path != "persistent":
        return None, None
    path = os.path.join(ROOT, "profiles", "decode_persist_traffic.json")
    try:
        with open(path) as f:
            prof = json.load(f)
        return prof["hbm_bytes_per_launch"], prof.get("kernel_source_sha256_16") == source_hash()
    except (OSError, KeyError, ValueError):
        return None, None


def prefill_heavy(H, synth, g, cfg, seed):
    """The prefill-heavy workload: 4 prompts of 32 cond + 512 text ids (4 x 547 = 2188 rows)
    in one causal forward producing the logits of every row (kept on the device); median of
    3 calls after one warm-up, host call to return.  FLOPs are the algorithmic ones: the
    linears of every row (24 blocks + mel_head) and causal attention."""
    prompts = []
    for b in range(4):
        pr = synth.make_prompt(cfg, 32, 512, seed=seed + 10 + b)
        prompts.append(H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None))
    g.forward_logits(prompts, copy_out=False)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        g.forward_logits(prompts, copy_out=False)
        times.append((time.perf_counter() - t0) * 1e3)
    ms = statistics.median(times)
    d, F, V, L, rows, T = 1280, 5120, 8194, 24, 4 * 547, 547
    lin = 2.0 * rows * (L * (d * 3 * d + d * d + d * F + F * d) + d * V)
    att = 4 * L * 20 * (T * (T + 1) / 2) * 64 * 2 * 2
    tflop = (lin + att) / 1e12
    print(f"[bench] prefill-heavy forward: {ms:.2f} ms", file=sys.stderr, flush=True)
    return {"workload": "batch 4 x (32 cond + 512 text) = 2188 rows, one forward, logits of all rows",
            "ms": round(ms, 3), "tflop": round(tflop, 4), "achieved_tflops": round(tflop / (ms * 1e-3), 1),
            "bound": "mfma", "peak_tflops": 2500.0,
            "frac": round(tflop / (ms * 1e-3) / 2500.0, 4),
            "note": "fp16 MFMA with hi/lo split activations (two products per weight)"}


def short_decode(H, synth, g, cfg, seed):
    """The short workload (config 1): prefill 32 cond + 64 text (99 rows), 128 greedy steps
    (penalty 10, STOP masked), bf16 cache; median of 5 generations, host call time."""
    n_cond, n_text, n_steps, samp, bits, desc = WORKLOADS["short"]
    pr = synth.make_prompt(cfg, n_cond, n_text, seed=seed + 1)
    sp = H.SamplingParams(max_mel_tokens=n_steps, **samp)
    cp = H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, n_steps)
    kv = g.kv_cache(2048, H.ITTS_BF16)
    H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(0))
    times, steps = [], []
    for _ in range(5):
        t0 = time.perf_counter()
        codes = H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(0))
        times.append((time.perf_counter() - t0) * 1e3)
        t = kv.last_timing()
        steps.append(t["decode_ms"] / t["decode_steps"])
    ms = statistics.median(times)
    print(f"[bench] short decode: {n_steps / (ms * 1e-3):.1f} tokens/s", file=sys.stderr, flush=True)
    return {"workload": desc, "tokens": len(codes), "ms": round(ms, 3),
            "tokens_per_s": round(n_steps / (ms * 1e-3), 1),
            "decode_step_us": round(statistics.median(steps) * 1e3, 2)}


def f32_kv_decode(H, g, cp, sp, weight_bytes):
    """The long workload with the reference's fp32 cache instead of bf16 (twice the KV
    bytes per key): one warm-up and one timed generation, device-timed decode rate."""
    kv = g.kv_cache(2048, H.ITTS_F32)
    path = "persistent" if kv.decode_path() == H.ITTS_DECODE_PERSISTENT else "multi-kernel"
    H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(1234))
    codes = H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(1234))
    t = kv.last_timing()
    step_ms = t["decode_ms"] / t["decode_steps"]
    mean_L = int(round(t["prefill_rows"] + (t["decode_steps"] + 1) / 2.0))
    nbytes = step_bytes(weight_bytes, mean_L) + KV_ROW_BYTES * (mean_L + 1)  # f32 rows: twice bf16's
    achieved = nbytes / (step_ms * 1e-3) / 1e9
    print(f"[bench] f32-cache decode: {1e3 / step_ms:.1f} tokens/s ({path})", file=sys.stderr, flush=True)
    kv.close()
    return {"workload": "the long workload with an fp32 KV cache", "decode_path": path, "tokens": int(len(codes)),
            "decode_tokens_per_s": round(1e3 / step_ms, 2), "decode_step_us": round(step_ms * 1e3, 2),
            "hbm_achieved_gbs": round(achieved, 1), "hbm_frac": round(achieved / HBM_PEAK_GBS, 4)}


def batch_decode(H, synth, g, cfg, seed, weight_bytes):
    """The batched workload: 8 sentences with text lengths U[20, 200] and decode lengths
    U[200, 1200] (seeded), each stopping at its own length (STOP masked until then),
    sampled (T 0.8, top-k 30, top-p 0.8, penalty 10), bf16 caches of 2048 rows.  One
    generate_codes_batch call: 8 prefills, then one batched step per token while any
    sequence runs.  Aggregate rate = all generated tokens / host call time."""
    rng = np.random.default_rng(seed + 100)
    n_text = rng.integers(20, 201, 8)
    n_dec = rng.integers(200, 1201, 8)
    prompts, params = [], []
    for b in range(8):
        pr = synth.make_prompt(cfg, 32, int(n_text[b]), seed=seed + 200 + b)
        prompts.append(H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, int(n_dec[b])))
        params.append(H.SamplingParams(greedy=False, temperature=0.8, top_k=30, top_p=0.8,
                                       repetition_penalty=10.0, max_mel_tokens=int(n_dec[b])))
    caches = [g.kv_cache(2048, H.ITTS_BF16) for _ in range(8)]
    H.generate_codes_batch(g, prompts, caches, params, [H.SamplerRng(b) for b in range(8)])
    t0 = time.perf_counter()
    codes = H.generate_codes_batch(g, prompts, caches, params, [H.SamplerRng(b) for b in range(8)])
    wall = time.perf_counter() - t0
    total = sum(len(c) for c in codes)
    assert [len(c) for c in codes] == [int(x) for x in n_dec]
    steps = int(n_dec.max())
    # the 8 prefills alone (the same prompts, host call time), so that the decode part of the
    # call can be priced against HBM
    t0 = time.perf_counter()
    for b in range(8):
        g.prefill(prompts[b].text_tokens, prompts[b].conds, prompts[b].lang_id, caches[b], logits=False)
    prefill_s = time.perf_counter() - t0
    decode_s = wall - prefill_s
    # Algorithmic bytes of the batched steps: sequence b (prompt rows T_b = 32 + n_text + 3)
    # makes n_dec - 1 steps, step i at T_b + i + 1 keys; every batched step streams the
    # weights once, and each live sequence reads its K/V rows, writes one and its logits.
    wb = weight_bytes
    Tb = 32 + n_text + 3
    n_steps = n_dec - 1
    n_batched = int(n_steps.max())
    kv_read = sum(KV_ROW_BYTES * (int(n_steps[b]) * int(Tb[b]) + int(n_steps[b]) * (int(n_steps[b]) + 1) // 2)
                  for b in range(8))
    per_seq_rest = (KV_ROW_BYTES + 8194 * 4) * int(n_steps.sum())
    total_bytes = n_batched * wb + kv_read + per_seq_rest
    gbs = total_bytes / decode_s / 1e9
    print(f"[bench] batch-8 decode: {total / wall:.1f} tokens/s aggregate, {gbs:.0f} GB/s", file=sys.stderr,
          flush=True)
    return {"workload": "batch 8 sentences, text lengths U[20,200], decode lengths U[200,1200] with per-sequence "
                        "stop, sampled (T 0.8, top-k 30, top-p 0.8, penalty 10), bf16 caches of 2048 rows",
            "text_lengths": [int(x) for x in n_text], "decode_lengths": [int(x) for x in n_dec],
            "tokens": total, "ms": round(wall * 1e3, 2),
            "aggregate_tokens_per_s": round(total / wall, 1),
            "per_sequence_tokens_per_s": round(steps / wall, 1),
            "prefills_ms": round(prefill_s * 1e3, 2), "decode_ms": round(decode_s * 1e3, 2),
            "batched_steps": n_batched, "algorithmic_bytes": int(total_bytes),
            "weight_bytes": int(n_batched * wb), "kv_read_bytes": int(kv_read),
            "hbm_achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "note": "host call time includes the 8 prefills; one batched step per token of the longest sequence; "
                    "hbm figures: algorithmic bytes of the batched steps (weights once per step, each live "
                    "sequence's K/V rows) / (call time - the 8 prefills' time)"}


def int4_decode(H, synth, seed):
    """The int4 workload: 4-bit weights, prefill 32 + 128 text (163 rows), 1500 greedy
    steps with STOP masked; device-timed decode rate and the HBM roofline of one step."""
    n_cond, n_text, n_steps, samp, bits, desc = WORKLOADS["int4"]
    cfg = dict(synth.FULL_CONFIG, quant_bits=bits)
    W = synth.make_weights(cfg, seed=seed)
    wb = W.weight_bytes_per_step()
    g = H.Gpt(W)
    kv = g.kv_cache(2048, H.ITTS_BF16)
    path = "persistent" if kv.decode_path() == H.ITTS_DECODE_PERSISTENT else "multi-kernel"
    prompt = synth.make_prompt(cfg, n_cond, n_text, seed=seed + 1)
    sp = H.SamplingParams(max_mel_tokens=n_steps, **samp)
    cp = H.CodePrompt(prompt.text_tokens, prompt.conds, prompt.lang_id, None, n_steps)
    H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(1))
    codes = H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(1))
    t = kv.last_timing()
    step_ms = t["decode_ms"] / t["decode_steps"]
    mean_L = t["prefill_rows"] + (t["decode_steps"] + 1) / 2.0
    achieved = step_bytes(wb, int(round(mean_L))) / (step_ms * 1e-3) / 1e9
    print(f"[bench] int4 decode: {1e3 / step_ms:.1f} tokens/s ({path})", file=sys.stderr, flush=True)
    g.close()
    return {"workload": desc, "decode_path": path, "tokens": int(len(codes)),
            "decode_tokens_per_s": round(1e3 / step_ms, 2), "decode_step_us": round(step_ms * 1e3, 2),
            "prefill_ms": round(t["prefill_ms"], 3), "weight_bytes_per_step": wb,
            "hbm_achieved_gbs": round(achieved, 1), "hbm_frac": round(achieved / HBM_PEAK_GBS, 4)}


def cfm_flops(c: dict, B: int, T: int) -> float:
    """Algorithmic FLOPs of one forward_merged over B x T rows (2 per multiply-add): the
    linears, WaveNet's convolutions and the attention products."""
    d, F, C_, L, NL, K = c["dim"], c["inter"], c["in_ch"], c["n_layers"], c["wn_layers"], c["wn_kernel"]
    R = B * T
    md = 2 * C_ + d + c["style_dim"]
    f = 2.0 * R * md * d
    f += L * 2.0 * R * d * (3 * d + d + 2 * F) + L * 2.0 * R * F * d + L * 4.0 * B * T * T * d
    f += (L - 1 - L // 2) * 2.0 * R * 2 * d * d
    f += 2.0 * R * (d + C_) * d + 2.0 * R * d * d
    f += sum(2.0 * R * K * d * 2 * d + 2.0 * R * d * (d if i + 1 == NL else 2 * d) for i in range(NL))
    f += 2.0 * R * d * d * 2 + 2.0 * R * d * C_
    return f


def cfm_solve(seed):
    """The Stage-2 CFM estimator (cfm.rs, reference shape: dim 512, 13 layers, 8 heads,
    SwiGLU 1536, WaveNet 8 x kernel 5) in its 25-step Euler solve with CFG 0.7 for 10 s of
    audio: 861 generated frames (22,050 Hz / hop 256 = 86.13 frames/s) after a 172-frame
    prompt (the reference fixture's ref_mel), T_total 1033, the CFG pair as batch 2.  The
    reference's figure for the same stage and audio length is 1,540 ms (M-series GPU,
    docs/benchmarks/indextts-rust-verification-and-benchmark-report.md:135)."""
    from itts_hip import synth
    from itts_hip.cfm import FULL_CONFIG, CfmDit
    W = synth.make_cfm_weights(FULL_CONFIG, seed=seed)
    m = CfmDit(W, FULL_CONFIG)
    inp = synth.make_cfm_inputs(FULL_CONFIG, 1033, 172, seed=seed)
    args = (inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], 25, 0.7)
    m.solve_euler(*args)
    walls, devs = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        m.solve_euler(*args)
        walls.append((time.perf_counter() - t0) * 1e3)
        devs.append(m.last_timing_ms())
    m.close()
    dev = statistics.median(devs)
    tflop = 25 * cfm_flops(FULL_CONFIG, 2, 1033) / 1e12
    print(f"[bench] CFM 25-step solve (10 s of audio): {dev:.1f} ms device, {statistics.median(walls):.1f} ms host",
          file=sys.stderr, flush=True)
    return {"workload": "CFM DiT 25-step Euler solve, CFG 0.7, T_total 1033 (172 prompt + 861 generated frames = "
                        "10 s of audio), batch 2 (CFG pair), fp32, seeded weights of the reference shape",
            "solve_ms": round(dev, 2), "host_call_ms": round(statistics.median(walls), 2),
            "reference_ms": 1540.0, "speedup_vs_reference": round(1540.0 / dev, 2),
            "tflop_per_solve": round(tflop, 3), "achieved_tflops": round(tflop / (dev * 1e-3), 1),
            "peak_tflops": 833.3, "frac": round(tflop / (dev * 1e-3) / 833.3, 4),
            "note": "fp32 activations; linears, WaveNet convolutions and attention on fp16 hi/lo split MFMA "
                    "(three fp16 products per product, fp32 accumulation); peak = fp16 dense 2.5 PFLOP/s / 3"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="long", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-steps", type=int, default=30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the prefill-heavy (4 x 547 rows) and int4 decode measurements")
    ap.add_argument("--only", choices=["decode", "prefill", "prefill-heavy", "batch8", "cfm"],
                    help="for profilers: only repeat the workload's whole generation (decode), its "
                         "prefill or the prefill-heavy forward --repeat times, print one line per "
                         "call, no JSON")
    ap.add_argument("--repeat", type=int, default=6)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--decode", default="auto", choices=["auto", "multi", "persistent"],
                    help="decode-step implementation (auto: persistent where supported)")
    ap.add_argument("--kv", default="bf16", choices=["bf16", "f32"],
                    help="KV cache rows for --only decode / prefill")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the decoder runs one sequence per GPU and this "
              "build has no multi-GPU path (requests shard by sequence). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import itts_hip as H
    from itts_hip import synth

    n_cond, n_text, n_steps, samp, bits, desc = WORKLOADS[args.workload]
    cfg = dict(synth.FULL_CONFIG, quant_bits=bits)
    t0 = time.perf_counter()
    W = synth.make_weights(cfg, seed=args.seed)
    weight_bytes = W.weight_bytes_per_step()
    print(f"[bench] weights generated in {time.perf_counter() - t0:.1f}s "
          f"({weight_bytes / 1e6:.1f} MB per decode step)", file=sys.stderr, flush=True)
    g = H.Gpt(W)
    if args.only:
        prompt = synth.make_prompt(cfg, n_cond, n_text, seed=args.seed + 1)
        kv = g.kv_cache(2048, H.ITTS_BF16 if args.kv == "bf16" else H.ITTS_F32)
        heavy = []
        for b in range(4):
            pr = synth.make_prompt(cfg, 32, 512, seed=args.seed + 10 + b)
            heavy.append(H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None))
        if args.only == "cfm":
            r = cfm_solve(args.seed)
            print(f"[bench] cfm: {r['solve_ms']} ms per 25-step solve", flush=True)
            return
        if args.only == "batch8":
            r = batch_decode(H, synth, g, cfg, args.seed, weight_bytes)
            print(f"[bench] batch8: {r['aggregate_tokens_per_s']} tokens/s aggregate", flush=True)
            return
        if args.only == "decode":
            sp = H.SamplingParams(max_mel_tokens=n_steps, **samp)
            cp = H.CodePrompt(prompt.text_tokens, prompt.conds, prompt.lang_id, None, n_steps)
            for i in range(args.repeat):
                t0 = time.perf_counter()
                codes = H.generate_codes_after(g, cp, kv, sp, H.SamplerRng(1234))
                print(f"[bench] decode generation {i}: {len(codes)} codes in "
                      f"{(time.perf_counter() - t0) * 1e3:.2f} ms", flush=True)
            return
        for i in range(args.repeat):
            t0 = time.perf_counter()
            if args.only == "prefill":
                g.prefill(prompt.text_tokens, prompt.conds, prompt.lang_id, kv, logits=False)
            else:
                g.forward_logits(heavy, copy_out=False)
            print(f"[bench] {args.only} call {i}: {(time.perf_counter() - t0) * 1e3:.2f} ms", flush=True)
        return
    g.set_decode_path({"auto": H.ITTS_DECODE_AUTO, "multi": H.ITTS_DECODE_MULTI,
                       "persistent": H.ITTS_DECODE_PERSISTENT}[args.decode])
    kv = g.kv_cache(2048, H.ITTS_BF16)
    decode_path = "persistent" if kv.decode_path() == H.ITTS_DECODE_PERSISTENT else "multi-kernel"
    print(f"[bench] decode step: {decode_path}", file=sys.stderr, flush=True)
    prompt = synth.make_prompt(cfg, n_cond, n_text, seed=args.seed + 1)
    sp = H.SamplingParams(max_mel_tokens=n_steps, **samp)
    cp = H.CodePrompt(prompt.text_tokens, prompt.conds, prompt.lang_id, None, n_steps)
    hp = hip()

    def generate():
        rng = H.SamplerRng(1234)
        return H.generate_codes_after(g, cp, kv, sp, rng)

    for _ in range(args.warmup):
        codes = generate()
        print(f"[bench] warmup generation: {len(codes)} codes", file=sys.stderr, flush=True)

    # time to first token: host call -> first token id on the host (prefill + one sample)
    sp1 = H.SamplingParams(max_mel_tokens=1, **samp)
    ttft = []
    for _ in range(5):
        t0 = time.perf_counter()
        H.generate_codes_after(g, H.CodePrompt(prompt.text_tokens, prompt.conds, prompt.lang_id, None, 1),
                               kv, sp1, H.SamplerRng(1234))
        ttft.append((time.perf_counter() - t0) * 1e3)
    ttft_ms = statistics.median(ttft)

    ev0, ev1 = C.c_void_p(), C.c_void_p()
    hp.hipEventCreate(C.byref(ev0))
    hp.hipEventCreate(C.byref(ev1))
    stream = C.c_void_p(g.stream)
    hp.hipDeviceSynchronize()
    timings = []
    t0 = time.perf_counter()
    hp.hipEventRecord(ev0, stream)
    for _ in range(args.steps):
        codes = generate()
        timings.append(kv.last_timing())
    hp.hipEventRecord(ev1, stream)
    hp.hipEventSynchronize(ev1)
    hp.hipDeviceSynchronize()
    wall = time.perf_counter() - t0
    region_ms = C.c_float()
    hp.hipEventElapsedTime(C.byref(region_ms), ev0, ev1)
    n_tok = len(codes)
    assert n_tok == n_steps, (n_tok, n_steps)

    T = timings[-1]["prefill_rows"]
    dec_steps = timings[-1]["decode_steps"]
    dec_ms = statistics.mean(t["decode_ms"] for t in timings)
    pre_ms = statistics.mean(t["prefill_ms"] for t in timings)
    step_ms = dec_ms / dec_steps
    mean_L = T + (dec_steps + 1) / 2.0  # keys of step i: T + i + 1, i = 0..dec_steps-1
    bytes_step = step_bytes(weight_bytes, int(round(mean_L)))

    # The dominant kernel alone: the same decode steps (contexts T+1 .. T+dec_steps, so the
    # same mean context) launched back to back between HIP events on the decoder's stream.
    g.prefill(prompt.text_tokens, prompt.conds, prompt.lang_id, kv, logits=False)
    kernel_ms = kv.decode_timing(100, 2, dec_steps)
    achieved = bytes_step / (kernel_ms * 1e-3) / 1e9
    kernel_name = ("decode_persist_kernel (one launch = one decode step)" if decode_path == "persistent"
                   else "decode step (122 kernels)")
    traffic, traffic_current = measured_traffic(decode_path)
    value = args.steps * n_tok / wall
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded random-init weights of the reference architecture)",
        "config": {"workload": desc, "weights": f"int{bits} MLX-affine group 64, fp16 params",
                   "kv_cache": "bf16", "layers": 24, "d_model": 1280, "heads": 20,
                   "prefill_rows": T, "decode_tokens": n_tok, "step": "one full generation",
                   "decode_path": decode_path},
        "ttft_ms": round(ttft_ms, 3),
        "ttft": ttft_roofline(ttft_ms, pre_ms, T, weight_bytes),
        "decode_tokens_per_s": round(dec_steps / (dec_ms * 1e-3), 2),
        "decode_step_us": round(step_ms * 1e3, 2),
        "prefill_ms": round(pre_ms, 3),
        "gpu_region_ms": round(region_ms.value, 3),
        "decode_kernel_us": round(kernel_ms * 1e3, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_measured_on_this_kernel_source": traffic_current,
                     "kernel": kernel_name,
                     "bytes_per_launch": bytes_step, "mean_keys": mean_L},
    }
    if not args.no_secondary and args.workload == "long":
        out["secondary"] = {"short_decode": short_decode(H, synth, g, cfg, args.seed),
                            "f32_kv_decode": f32_kv_decode(H, g, cp, sp, weight_bytes),
                            "prefill_heavy": prefill_heavy(H, synth, g, cfg, args.seed),
                            "batch8_decode": batch_decode(H, synth, g, cfg, args.seed, weight_bytes)}
        del g, kv
        out["secondary"]["int4_decode"] = int4_decode(H, synth, args.seed)
        out["secondary"]["cfm_solve"] = cfm_solve(args.seed)
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (oracle) ...", file=sys.stderr, flush=True)
        n_prior = max(0, int(round(mean_L)) - T)
        out["cpu_baseline"] = cpu_baseline(W, prompt, sp, args.cpu_steps, codes[:n_prior])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
