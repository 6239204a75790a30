"""Per-phase timeline of one layer of the persistent decode step on every block, from the
instrumented library (build.sh).  Full-size synthetic decoder, a 32 + 200 prompt with prior
codes so that the traced step attends over about 985 keys (the long workload's mean
context), layer 12 (mid-stack); the stamps of a few warm steps are discarded.

Usage (repository root): python3 index-tts-rs_amd/trace/phase_trace.py [--layer L] [--prior P]
Prints a markdown table: per phase, the time from the earliest block's layer start at
which the blocks passed it (min / median / max over blocks) and the median phase length.
"""
import argparse
import ctypes as C
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
os.environ["ITTS_HIP_LIB"] = os.path.join(HERE, "lib", "libitts_trace.so")
sys.path.insert(0, os.path.dirname(HERE))
import numpy as np  # noqa: E402
import itts_hip as H  # noqa: E402
from itts_hip import synth  # noqa: E402

PHASES = [(0, "layer start"), (1, "x all-gather in"), (2, "QKV dot + LN1 statistics"), (3, "QKV row sums"),
          (4, "q/k/v in (attention blocks)"), (5, "scores"), (6, "P.V"), (9, "attention all-gather in"),
          (10, "c_proj dot"), (11, "c_proj row sums + residual"), (12, "x_mid all-gather in"),
          (13, "c_fc dot + LN2 statistics"), (14, "c_fc row sums + GELU"), (15, "x_f all-gather in"), (16, "mlp c_proj dot"),
          (17, "mlp row sums + residual")]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layer", type=int, default=12)
    ap.add_argument("--prior", type=int, default=750)
    args = ap.parse_args()
    W = synth.make_weights(synth.FULL_CONFIG, seed=11)
    g = H.Gpt(W)
    pr = synth.make_prompt(W.cfg, 32, 200, seed=2)
    rd = H.lib.itts_trace_read
    rd.argtypes = [C.c_void_p, C.c_int]
    buf = np.zeros((1024, 32), np.uint64)
    kv = g.kv_cache(2048)
    assert kv.decode_path() == H.ITTS_DECODE_PERSISTENT
    g.prefill_after(pr.text_tokens, pr.conds, pr.lang_id, np.arange(args.prior, dtype=np.int32) % 8000, kv)
    pos = args.prior + 1  # mel position of the next code (the prompt's start code is position 0)
    for _ in range(4):  # warm steps
        rd(buf.ctypes.data, args.layer)
        g.step(kv, 5, pos)
        pos += 1
    rd(buf.ctypes.data, args.layer)
    g.step(kv, 5, pos)
    rd(buf.ctypes.data, args.layer)
    t = buf.astype(np.int64)
    live = t[:, 0] > 0
    t0 = t[live, 0].min()
    print(f"Layer {args.layer}, step attending over {kv.valid_len()} keys, {int(live.sum())} blocks; "
          f"times in us from the earliest block's layer start (100 MHz counter)\n")
    print("| Phase (stamp after) | blocks | min | median | max | median length |")
    print("|---|---|---|---|---|---|")
    prev = None
    for i, name in PHASES:
        col = t[:, i]
        ok = col > 0
        rel = (col[ok] - t0) * 0.01
        med = float(np.median(rel))
        length = "" if prev is None else f"{med - prev:.2f}"
        print(f"| {name} | {int(ok.sum())} | {rel.min():.2f} | {med:.2f} | {rel.max():.2f} | {length} |")
        prev = med
    clk = (t[live, 25] - t[live, 24]) / ((t[live, 17] - t[live, 0]) * 0.01)
    print(f"\nShader clock over the layer (s_memtime / s_memrealtime): median {np.median(clk):.0f} MHz")


if __name__ == "__main__":
    main()
