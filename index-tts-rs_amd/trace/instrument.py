"""Per-phase timeline of the persistent decode step: generates an instrumented copy of
csrc/kernels_persist.hip in which thread 0 of every block stamps the 100 MHz real-time
counter (s_memrealtime) at the phase barriers of one chosen layer, with
itts_trace_read() to copy the stamps out and choose the next traced layer.

Slots (per block): 0 layer start, 1 x in (poll done), 2 QKV dot (and the folded LN1's
statistics), 3 QKV row sums, 4 q/k/v in, 5 scores, 6 P.V, 9 attention in, 10 c_proj dot,
11 c_proj row sums, 12 x_mid in, 13 c_fc dot (and LN2's statistics), 14 c_fc row sums
(GELU), 15 x_f in, 16 mlp c_proj dot, 17 mlp row sums; 24 / 25 the shader clock (s_memtime) at slots 0 / 17; 26-28 and
29-31 the first loader lane and the publisher around the QKV and c_fc dots.

Usage: python3 instrument.py <kernels_persist.hip> <out.hip>; build.sh builds the library.
"""
import re
import sys

src, dst = sys.argv[1], sys.argv[2]
s = open(src).read()


def once(old, new):
    global s
    assert s.count(old) == 1, old[:70]
    s = s.replace(old, new)


def stamp_after(pattern, idx):
    global s
    m = re.search(pattern, s, re.S)
    assert m, pattern
    s = s[: m.end()] + f"\n    STAMP({idx});" + s[m.end():]


once('namespace itts {\n\nnamespace {\n',
     'namespace itts {\nconstexpr int kTraceBlocks = 1024;\n__device__ unsigned long long g_trace[kTraceBlocks][32];\n__device__ int g_trace_layer;\nnamespace {\n')
once('#include "kernels.h"',
     '#include "kernels.h"\n#define STAMP(i) do { if (T == 0 && l == g_trace_layer && b < 1024) '
     'g_trace[b][i] = __builtin_amdgcn_s_memrealtime(); } while (0)')
once("// ---------------- P1: LN1 (folded), QKV rows; K/V rows into the cache ------------",
     "// ---------------- P1: LN1 (folded), QKV rows; K/V rows into the cache ------------\n    STAMP(0);\n"
     "    if (T == 0 && l == g_trace_layer && b < 1024) g_trace[b][24] = __builtin_amdgcn_s_memtime();")
stamp_after(r"\] = lp\[i\] \* xin\[i\];\s*\}\s*__syncthreads\(\);\s*if \(sh\.abort\) return;", 1)
stamp_after(r"dot_slots<BITS>\(wq, m_qkv, xn, part, ll\);(?:\s*//[^\n]*)*\s*if \(loader && l > 0\) load_slots<BITS, PT>\(wp, Ly\.proj, m_proj, ll\);\s*__syncthreads\(\);", 2)
stamp_after(r"lp\[bo_cq \+ r\]; \}\);\s*\}\s*__syncthreads\(\);", 3)
stamp_after(r"if \(!ok\) sh\.abort = 1;\s*\}\s*__syncthreads\(\);\s*if \(sh\.abort\) return;", 4)
stamp_after(r"if \(lane == 0\) sh\.m_w\[lw\] = mloc;\s*\}\s*__syncthreads\(\);", 5)
stamp_after(r"if \(lane == 0\) sh\.l_w\[lw\] = lsum;\s*\}\s*__syncthreads\(\);", 6)
stamp_after(r"xin\[xpad<BITS>\(h \* 64 \+ 3 \* j \+ e\)\] = f\[e\];\s*\}\)\)\s*sh\.abort = 1;\s*__syncthreads\(\);"
            r"\s*if \(sh\.abort\) return;", 9)
stamp_after(r"dot_slots<BITS>\(wp, m_proj, xin, part, ll\);\s*__syncthreads\(\);", 10)
stamp_after(r"out\[r\] = xm;\s*\}\);\s*__syncthreads\(\);", 11)
stamp_after(r"poll_rows_ln<BITS>\(a\.x_mid, [^;]*\) sh\.abort = 1;\s*__syncthreads\(\);"
            r"\s*if \(sh\.abort\) return;", 12)
stamp_after(r"dot_slots<BITS>\(wf, m_fc, xn, part, ll\);\s*__syncthreads\(\);", 13)
stamp_after(r"lp\[bo_cf \+ r\]\); \}\);\s*\}\s*__syncthreads\(\);", 14)
stamp_after(r"poll_rows<BITS, true>\(a\.x_f, [^;]*\) sh\.abort = 1;[^\n]*\s*__syncthreads\(\);\s*if \(sh\.abort\) return;", 15)
stamp_after(r"dot_slots<BITS>\(wm, m_mp, xin, part, ll\);\s*__syncthreads\(\);", 16)
stamp_after(r"own\[r\] = xo;\s*out\[r\] = xo;\s*\}\);\s*__syncthreads\(\);", 17)
once("    STAMP(17);", "    STAMP(17);\n    if (T == 0 && l == g_trace_layer && b < 1024) g_trace[b][25] = __builtin_amdgcn_s_memtime();")
for dot, i0 in (("wq, m_qkv, xn", 26), ("wf, m_fc, xn", 29)):
    once(f"    if (loader) dot_slots<BITS>({dot}, part, ll);",
         f"    if (T == 448 && l == g_trace_layer && b < 1024) g_trace[b][{i0}] = __builtin_amdgcn_s_memrealtime();\n"
         f"    if (loader) dot_slots<BITS>({dot}, part, ll);\n"
         f"    if (T == 448 && l == g_trace_layer && b < 1024) g_trace[b][{i0 + 1}] = __builtin_amdgcn_s_memrealtime();\n"
         f"    if (T == 384 && l == g_trace_layer && b < 1024) g_trace[b][{i0 + 2}] = __builtin_amdgcn_s_memrealtime();")
once("}  // namespace itts", """}  // namespace itts
extern "C" int itts_trace_read(unsigned long long *host, int layer_next) {
  if (hipMemcpyFromSymbol(host, HIP_SYMBOL(itts::g_trace), sizeof(itts::g_trace)) != hipSuccess) return 1;
  if (hipMemcpyToSymbol(HIP_SYMBOL(itts::g_trace_layer), &layer_next, sizeof(int)) != hipSuccess) return 2;
  return 0;
}""")
open(dst, "w").write(s)
print("instrumented:", s.count("STAMP(") - 1, "phase stamps")
