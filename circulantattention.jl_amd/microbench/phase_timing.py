"""Per-wave phase timing of the split-half fused kernels at cfg3 (or cfg5).

A copy of libcircatt built with CIRCATT_F2H_PHASE=1 makes every wave of
kernel2h sum s_memtime spans of four phases over its items (staging, the two
barriers, the walk with its epilogue) and lets the waves of workgroups 0..7
write the sums to a buffer of 512 floats given to that copy's extra entry
point circatt_debug_set_phase_buffer.  This script builds that copy (on a
machine with hipcc; the other objects come from the in-tree build) and, on an
MI355X, runs the three cfg3 kernels and prints the phases per wave slot.

    python circulantattention.jl_amd/microbench/phase_timing.py --build [--no-prio]
    python circulantattention.jl_amd/microbench/phase_timing.py [--no-prio]

--no-prio builds and runs a second copy with CIRCATT_F2H_PRIO=0 (equal wave
priorities over the walk).  --config cfg5 does the same for the kernels of 32
real components per head (8 wavefronts per workgroup) at cfg5's shape.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
F2H16 = ("fused2h_fwd.hip", "fused2h_bwdq.hip", "fused2h_bwdkv.hip")
F2H32 = ("fused2h2_fwd.hip", "fused2h2_bwdq.hip", "fused2h2_bwdkv.hip")
F1H32 = ("fused1h2_fwd.hip", "fused1h2_bwdq.hip", "fused1h2_bwdkv.hip")
# name: (spatial n1, n2, channels, batch, heads, window, complex, sources, waves per workgroup,
#        spatial dims, similarity kind)
CONFIGS = {"cfg3": (256, 256, 64, 4, 4, 15, False, F2H16, 16, 2, 0),
           "cfg5": (320, 320, 32, 2, 2, 11, True, F2H32, 8, 2, 0),
           "cfg4b": (262144, 1, 32, 2, 1, 63, False, F1H32, 8, 1, 1)}
F2H = F2H16


def lib_path(no_prio: bool) -> str:
    tag = "" if F2H is F2H16 else "32" if F2H is F2H32 else "1d"
    return os.path.join(HERE, f"libcircatt_phase{tag}_noprio.so" if no_prio else f"libcircatt_phase{tag}.so")


def build(no_prio: bool) -> None:
    sys.path.insert(0, PKG)
    import build as B

    B.build()  # the in-tree objects the copy links against
    objs = [os.path.join(B.OBJ, os.path.splitext(s)[0] + ".o") for s in B.SOURCES
            if s not in F2H]
    out = []
    for src in F2H:
        o = os.path.join(HERE, os.path.splitext(src)[0] + ("_np" if no_prio else "") + "_phase.o")
        defs = ["-DCIRCATT_F2H_PHASE=1"] + (["-DCIRCATT_F2H_PRIO=0"] if no_prio else [])
        subprocess.run([B.HIPCC, *B.FLAGS, *defs, "-c",
                        os.path.join(B.CSRC, src), "-o", o], check=True)
        out.append(o)
    lib = lib_path(no_prio)
    subprocess.run([B.HIPCC, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-o", lib,
                    *out, *objs], check=True)
    for o in out:
        os.remove(o)
    print("built", lib)


def run(no_prio: bool) -> None:
    import torch  # before the library: the process then uses torch's HIP runtime

    sys.path.insert(0, PKG)
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr

    lib = ctypes.CDLL(lib_path(no_prio))
    for name, (res, args) in L.SIGNATURES.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    n1, n2, C, B, nh, ws, cplx, _, nw, nsp, kind = CONFIGS[CFG]
    P = n1 * n2
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1003)
    shape = (B, C, n2, n1) if nsp == 2 else (B, C, n1)
    dt, DT = (torch.complex64, L.C32) if cplx else (torch.float32, L.F32)
    q, k, v, dy = (torch.randn(shape, device=dev, generator=g, dtype=dt) for _ in range(4))
    yb, dqb, dkb, dv = (torch.empty_like(q) for _ in range(4))
    phase = torch.zeros(8 * 16 * 4, device=dev)
    lib.circatt_debug_set_phase_buffer.restype = None
    lib.circatt_debug_set_phase_buffer.argtypes = [ctypes.c_void_p]
    lib.circatt_debug_set_phase_buffer(ptr(phase))
    lse = torch.empty((B * nh, P), device=dev)
    wb = lib.circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nh, B)
    work = torch.empty((wb // 4,), device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def fwd():
        L.check(lib.circatt_fused_fwd(kind, DT, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                      ptr(yb), ptr(lse), s))

    def bwd_dq():
        L.check(lib.circatt_fused_bwd_dq(kind, DT, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                         ptr(yb), ptr(dy), ptr(lse), ptr(dqb), ptr(work), wb, s))

    def bwd_dkdv():
        L.check(lib.circatt_fused_bwd_dkdv(kind, DT, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                           ptr(v), ptr(dy), ptr(lse), ptr(dkb), ptr(dv), ptr(work),
                                           wb, s))

    for _ in range(400):  # clocks to steady state
        fwd()
        bwd_dq()
        bwd_dkdv()
    torch.cuda.synchronize()
    print(f"{CFG}, cycles summed over each wave's items (mean over the 8 sampled workgroups)"
          + (", equal wave priorities" if no_prio else ""))
    for name, f in (("forward", fwd), ("query-centric", bwd_dq), ("key-centric", bwd_dkdv)):
        for _ in range(50):
            f()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        f()
        e1.record()
        torch.cuda.synchronize()
        t = phase.view(torch.int32).cpu().numpy().reshape(8, 16, 4)[:, :nw].astype("int64")
        tot = t.sum(axis=2)
        m = t.mean(axis=(0, 1))
        print(f"{name}: kernel {e0.elapsed_time(e1) * 1e3:.1f} us, "
              f"{tot.max() / (e0.elapsed_time(e1) * 1e-3) / 1e9:.2f} GHz (cycles / time)")
        print("  phases (mean over waves): staging %.0f, barrier after maxima %.0f, "
              "barrier after staging %.0f, walk+epilogue %.0f" % tuple(m))
        print(f"  walk+epilogue per wave slot 0..{nw - 1} (mean over workgroups):",
              [int(x) for x in t[:, :, 3].mean(axis=0)])


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--build", action="store_true")
    ap.add_argument("--no-prio", action="store_true")
    ap.add_argument("--config", choices=sorted(CONFIGS), default="cfg3")
    args = ap.parse_args()
    CFG = args.config
    F2H = CONFIGS[CFG][7]
    build(args.no_prio) if args.build else run(args.no_prio)
