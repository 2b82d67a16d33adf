"""Phase budget of one config-1 decode call from wall-clock stamps.

Developer measurement for the staged decode kernel and its merge: loads the
stamps build of the library (``make -C kaplumba_amd/csrc stamps`` builds
``kaplumba_amd/libkaplumba_tq_stamps.so``: the same sources with
-DTQ_PHASE_STAMPS), replays a HIP graph of config-1 calls over distinct layer
caches as bench.py does, and prints, for the last replayed call, the 100 MHz
wall clock (s_memrealtime) at each phase boundary of attn_stage_kernel
(per workgroup, or per wave) and attn_merge_rot_kernel, in microseconds.

    python3 kaplumba_amd/csrc/phase_stamps.py [--reps 3]
"""
import argparse
import ctypes
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from kaplumba_amd import _lib  # noqa: E402

NW = 8  # waves of the staged kernel


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--steps", type=int, default=200)
    args = ap.parse_args()
    _lib.LIB_PATH = os.path.join(ROOT, "kaplumba_amd", "libkaplumba_tq_stamps.so")
    lib = _lib.load()
    lib.tq_dbg_stage_stamps.argtypes = [ctypes.c_void_p, ctypes.c_longlong]
    lib.tq_dbg_merge_stamps.argtypes = [ctypes.c_void_p, ctypes.c_longlong]
    import bench
    from kaplumba_amd import ops

    dev = torch.device("cuda", 0)
    c = dict(bench.CFG1)
    n_layers = 24
    layers, kc, vc = bench.make_layer_caches(torch, n_layers, c, dev)
    g = torch.Generator(device=dev).manual_seed(1003)
    qs = [torch.randn(1, c["Hq"], 1, c["D"], device=dev, generator=g).to(torch.bfloat16)
          for _ in range(n_layers)]
    scale = 1.0 / math.sqrt(c["D"])

    def step(i):
        (kn, kp), (vn, vp) = layers[i % n_layers]
        return ops.attention_packed(qs[i % n_layers], kn, kp, vn, vp, kc, vc, scale, False)

    def q(x):
        return f"median {np.median(x):6.2f}  p90 {np.percentile(x, 90):6.2f}  max {x.max():6.2f}"

    for rep in range(args.reps):
        ms, outs, graph = bench.graph_timed(torch, step, args.steps, 20, dev)
        st = np.zeros((40, 1024), dtype=np.uint64)
        mt = np.zeros((4, 1024), dtype=np.uint64)
        assert lib.tq_dbg_stage_stamps(st.ctypes.data, st.nbytes) == 0
        assert lib.tq_dbg_merge_stamps(mt.ctypes.data, mt.nbytes) == 0
        st = st[:, :256].astype(np.int64)  # 32 splits x 8 kv heads
        mt = mt[:, :32].astype(np.int64)   # 4 rows x 8 kv heads
        t0 = st[0].min()
        a = lambda x: (x - t0) * 0.01  # noqa: E731
        e = st[0]
        r = lambda x: (x - e) * 0.01  # noqa: E731  (from the workgroup's own entry)
        print(f"== call time {ms * 1e3:.2f} us (graph of {args.steps} calls); "
              f"stamps of the last replayed call, us")
        print("  stage kernel, from each workgroup's entry:")
        print("    entry (from the first)     ", q(a(e)))
        print("    codebooks in registers     ", q(r(st[1])))
        print("    pair tables stored         ", q(r(st[2])))
        print("    query row in LDS           ", q(r(st[3])))
        print("    query rotated and staged   ", q(r(st[4])))
        print("    staging barrier            ", q(r(st[5])))
        print("    query operands loaded      ", q(r(st[6])))
        print("    loop start (per wave)      ", q(r(st[8:8 + NW]).ravel()))
        print("    first slot ready (per wave)", q(r(st[16:16 + NW]).ravel()))
        print("    loop end (per wave)        ", q(r(st[24:24 + NW]).ravel()))
        print("    loop length (per wave)     ", q(((st[24:24 + NW] - st[8:8 + NW]) * 0.01).ravel()))
        print("    wave spread in a workgroup ", q((st[24:24 + NW].max(0) - st[24:24 + NW].min(0)) * 0.01))
        le = st[24:24 + NW] - st[24:24 + NW].min(0)
        print("    loop end by wave index      " + " ".join(f"w{w} {np.median(le[w]) * 0.01:4.2f}" for w in range(NW)))
        ls = st[8:8 + NW] - st[8:8 + NW].min(0)
        print("    loop start by wave index    " + " ".join(f"w{w} {np.median(ls[w]) * 0.01:4.2f}" for w in range(NW)))
        print("    combine barrier            ", q(r(st[32])))
        print("    partial stored             ", q(r(st[33])))
        print("  absolute (from the first stage workgroup's entry):")
        print("    last partial stored        ", f"{a(st[33]).max():6.2f}")
        print("    merge entry                ", q(a(mt[0])))
        print("    merge loads in             ", q(a(mt[1])))
        print("    merge folded               ", q(a(mt[2])))
        print("    merge rows stored          ", q(a(mt[3])))
        print(f"    next call's first entry     {ms * 1e3:6.2f} (one call period)")
        del graph, outs


if __name__ == "__main__":
    main()
