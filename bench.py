"""Benchmark of the TurboQuant KV-cache hot path on one MI355X.

Default workload: decode attention over a 3-bit TurboQuant
cache, batch 1, one bf16 query token, 32 query heads / 8 kv heads, d=128,
32768 cached tokens per kv head, Hadamard rotation, Beta codebook, f32 norms.
A step is one attention call over one layer's cache; successive steps walk
over distinct layer caches (>= 512 MB in total) so the 256 MB Infinity Cache
cannot serve repeats.  The caches are written by the library's own append
kernel from seeded synthetic K/V (N(0,1) x per-channel log-normal(0, 0.5)).

The K timed steps are captured once in a HIP graph and replayed, bracketed by
HIP events on the replay stream, so the measurement is the GPU's time for
exactly K back-to-back attention calls (no Python launch overhead between
them); one replay is checked against the eager result first.  An attention
call is two kernels on that stream (the split-K partial kernel and the split
merge kernel), and the roofline figure is the call's time.

Prints one JSON line: value = algorithmic packed bytes per step / time per
step (GB/s); cpu_baseline = the numpy restatement of the reference algorithm
(oracle/) on a bounded sample, host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes one cfg1 attention call moves (both kernels), from rocprofv3
# FETCH_SIZE / WRITE_SIZE passes over this script scaled by the counters' reading
# of an elementwise kernel of known traffic (read x 1.9984, write x 1.0000); the
# counter runs and the calibration are summarised with the committed profiles.
CFG1_TRAFFIC_BYTES = 28_736_752
MFMA_BF16_PEAK_TFLOPS = 2500.0
CFG1 = dict(B=1, Hq=32, Hkv=8, D=128, T=32768, bits=3)
# config 2: ragged batched decode, d=256, K4/V2, dense 256x256 rotation
CFG2 = dict(B=32, Hq=16, Hkv=8, D=256, kb=4, vb=2, lo=2048, hi=8192, seed=1004)
# config 3: prefill append of one 8192-token chunk into a 36-layer cache
CFG3 = dict(layers=36, plain_layers=4, Hkv=8, T=8192, D=128, bits=3)
# config 4: speculative verify, 4 drafts per sequence, 131072 + 4 cached tokens, K2/V1
CFG4 = dict(B=4, Hq=32, Hkv=8, L=4, T=131072 + 4, D=128, kb=2, vb=1)
# prefill attention: one prefill_step_size chunk (256 queries) at the end of an
# 8192-token prompt, config-1 heads and widths, causal
CFGP = dict(B=1, Hq=32, Hkv=8, L=256, T=8192, D=128, bits=3)
CODEBOOK_NOTE = ("every leg uses the Beta Lloyd-Max codebooks the reference cache builds "
                 "(turboquant_cache.py:3587-3642); BASELINE's configs 0, 1 and 4 name the N(0,1) "
                 "Lloyd-Max codebook, which the kernels take as data at the same speed and which the "
                 "full-size GPU tests run against the oracle")


def algorithmic_decode_bytes(Hkv, T, D, kb, vb, norm_bytes, B=1):
    """Packed K + V index bytes and K + V norms read for one decode step."""
    pw_k = (D * kb + 31) // 32
    pw_v = (D * vb + 31) // 32
    return B * Hkv * T * (4 * pw_k + 4 * pw_v + 2 * norm_bytes)


def quantize_bytes(n_vec, D, bits, in_bytes, norm_bytes):
    """Raw input read + packed rows and norms written."""
    return n_vec * (D * in_bytes + 4 * ((D * bits + 31) // 32) + norm_bytes)


def make_layer_caches(torch, n_layers, c, dev):
    from kaplumba_amd import ops

    kc, vc = ops.Codec(c["D"], c["bits"], 0), ops.Codec(c["D"], c["bits"], 1)
    g = torch.Generator(device=dev)
    layers = []
    for i in range(n_layers):
        g.manual_seed(1000 + i)
        scale = torch.exp(torch.randn(1, c["Hkv"], 1, c["D"], device=dev, generator=g) * 0.5)
        st = []
        for codec in (kc, vc):
            x = (torch.randn(c["B"], c["Hkv"], c["T"], c["D"], device=dev, generator=g) * scale).half()
            pk = torch.empty((c["B"], c["Hkv"], c["T"], codec.packed_width), dtype=torch.uint32, device=dev)
            nm = torch.empty((c["B"], c["Hkv"], c["T"]), dtype=torch.float32, device=dev)
            ops.append_quantize(x, codec, pk, nm, 0)
            st.append((nm, pk))
            del x
        layers.append(st)
    torch.cuda.synchronize()
    return layers, kc, vc


def graph_timed(torch, step, steps, warmup, dev):
    """Capture `steps` calls of step(i) in a HIP graph and time one replay.

    Warm-up runs on the capture stream first, so that the library's
    per-stream workspace and the codec tables exist before capture (no
    allocation or memset is recorded into the graph).  Returns ms per step.
    """
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for i in range(max(warmup, 1)):
            step(i)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = [step(i) for i in range(steps)]
    with torch.cuda.stream(s):
        g.replay()  # upload + first execution, untimed
    torch.cuda.synchronize(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        e0.record(s)
        g.replay()
        e1.record(s)
    torch.cuda.synchronize(dev)
    return e0.elapsed_time(e1) / steps, outs, g


def bench_decode(torch, args, dev):
    from kaplumba_amd import ops

    c = dict(CFG1, T=args.tokens)
    per_layer = algorithmic_decode_bytes(c["Hkv"], c["T"], c["D"], c["bits"], c["bits"], 4)
    n_layers = max(2, math.ceil(args.rotate_mb * 1e6 / per_layer))
    layers, kc, vc = make_layer_caches(torch, n_layers, c, dev)
    g = torch.Generator(device=dev).manual_seed(1003)
    qs = [torch.randn(c["B"], c["Hq"], 1, c["D"], device=dev, generator=g).to(torch.bfloat16)
          for _ in range(n_layers)]
    scale = 1.0 / math.sqrt(c["D"])

    def step(i):
        (kn, kp), (vn, vp) = layers[i % n_layers]
        return ops.attention_packed(qs[i % n_layers], kn, kp, vn, vp, kc, vc, scale, False)

    ms, outs, graph = graph_timed(torch, step, args.steps, args.warmup, dev)
    # the replayed graph reproduces the eager calls (deterministic kernels)
    for i in (0, args.steps - 1):
        if not torch.equal(outs[i], step(i)):
            raise RuntimeError(f"graph replay of step {i} differs from the eager call")
    (kn, kp), (vn, vp) = layers[0]
    host = lambda t: t.cpu().numpy()
    sample = (qs[0].float().cpu().numpy(), host(kp), host(kn), host(vp), host(vn))
    return dict(bytes=per_layer, ms_per_step=ms, n_layers=n_layers,
                rotate_mb=n_layers * per_layer / 1e6, cpu_sample=sample)


def bench_floor(torch, dev, per_call, n_bufs):
    """The HBM floor the headline is read against, measured with the probe
    kernels of kaplumba_amd/libkaplumba_probe.so (roofline_probe.hip):

    * stream read: one launch reads `per_call` bytes (the cfg1 call's
      algorithmic bytes) with 16-byte nontemporal loads and writes nothing;
      launches walk `n_bufs` distinct buffers in a HIP graph, as the attention
      calls walk distinct layer caches; best of a small sweep of grid sizes
      and loads in flight.
    * device copy: 1 GiB copied (read + write counted), best of three grids.
    """
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "kaplumba_amd", "libkaplumba_probe.so"))
    lib.tqp_stream_read.restype = ctypes.c_int
    lib.tqp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p]
    lib.tqp_copy.restype = ctypes.c_int
    lib.tqp_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    bufs = [torch.empty(per_call, dtype=torch.uint8, device=dev) for _ in range(n_bufs)]
    for b in bufs:
        b.fill_(1)
    sink = torch.zeros(1 << 16, dtype=torch.uint32, device=dev)
    best = None
    for blocks in (256, 512, 1024, 2048):
        for unroll in (4, 8):
            def step(i, blocks=blocks, unroll=unroll):
                rc = lib.tqp_stream_read(bufs[i % n_bufs].data_ptr(), per_call, sink.data_ptr(), blocks,
                                         unroll, torch.cuda.current_stream(dev).cuda_stream)
                if rc:
                    raise RuntimeError(f"tqp_stream_read: HIP error {rc}")
            ms, _, _ = graph_timed(torch, step, 4 * n_bufs, 4, dev)
            if best is None or ms < best[0]:
                best = (ms, blocks, unroll)
    del bufs
    _free(torch)
    nbytes = 1 << 30
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    best_c = None
    for blocks in (1024, 4096, 16384):
        def cstep(_i, blocks=blocks):
            rc = lib.tqp_copy(src.data_ptr(), dst.data_ptr(), nbytes, blocks,
                              torch.cuda.current_stream(dev).cuda_stream)
            if rc:
                raise RuntimeError(f"tqp_copy: HIP error {rc}")
        ms, _, _ = graph_timed(torch, cstep, 5, 1, dev)
        if best_c is None or ms < best_c[0]:
            best_c = (ms, blocks)
    if not torch.equal(dst[:: 1 << 20], src[:: 1 << 20]):
        raise RuntimeError("tqp_copy: copy differs from its source")
    del src, dst
    _free(torch)
    ms, blocks, unroll = best
    return {"stream_read": {"bytes_per_launch": per_call, "us_per_launch": round(ms * 1e3, 3),
                            "GB/s": round(per_call / (ms * 1e-3) / 1e9, 2),
                            "launch": f"{blocks} x 256 threads, {unroll} 16-byte loads in flight per "
                                      f"thread, {n_bufs} distinct buffers in a HIP graph"},
            "device_copy": {"bytes": nbytes, "GB/s": round(2 * nbytes / (best_c[0] * 1e-3) / 1e9, 2),
                            "us": round(best_c[0] * 1e3, 2), "launch": f"{best_c[1]} x 256 threads",
                            "note": "read + write bytes"}}


def bench_quantize(torch, args, dev):
    """Config 0: append-quantize K and V f16 [1, 8, 4096, 128] at 3 bits (one layer)."""
    from kaplumba_amd import ops

    B, H, T, D, bits = 1, 8, 4096, 128, 3
    kc, vc = ops.Codec(D, bits, 0), ops.Codec(D, bits, 1)
    per_call = 2 * quantize_bytes(B * H * T, D, bits, 2, 4)
    n_sets = max(2, math.ceil(args.rotate_mb * 1e6 / per_call))
    g = torch.Generator(device=dev).manual_seed(1001)
    scale = torch.exp(torch.randn(1, H, 1, D, device=dev, generator=g) * 0.5)
    xs = [((torch.randn(B, H, T, D, device=dev, generator=g) * scale).half(),
           (torch.randn(B, H, T, D, device=dev, generator=g) * scale).half()) for _ in range(n_sets)]
    outs = [[(torch.empty((B, H, T, 12), dtype=torch.uint32, device=dev),
              torch.empty((B, H, T), dtype=torch.float32, device=dev)) for _ in range(2)]
            for _ in range(n_sets)]

    def step(i):  # the append of update_and_fetch: keys and values in one launch
        k, v = xs[i % n_sets]
        (kp, kn), (vp, vn) = outs[i % n_sets]
        ops.append_quantize_kv(k, v, kc, vc, kp, kn, vp, vn, 0)

    ms, _, _ = graph_timed(torch, step, args.steps, args.warmup, dev)
    return dict(bytes=per_call, ms_per_step=ms, kernel_bytes=per_call / 2)


def _free(torch):
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _synth_kv(torch, g, shape, dtype, dev):
    """N(0,1) x per-(kv head, channel) log-normal(0, 0.5) scales, like config 0."""
    B, H, T, D = shape
    scale = torch.exp(torch.randn(1, H, 1, D, device=dev, generator=g) * 0.5)
    return [(torch.randn(shape, device=dev, generator=g) * scale).to(dtype) for _ in range(2)]


def bench_ragged(torch, args, dev):
    """Config 2: 32 sequences of U[2048, 8192] tokens, d=256, K4/V2, dense rotation."""
    import numpy as np

    from kaplumba_amd import ops

    c = CFG2
    lens = np.random.default_rng(c["seed"]).integers(c["lo"], c["hi"] + 1, size=c["B"])
    cap = c["hi"]
    kc = ops.Codec(c["D"], c["kb"], 0, rotation="dense")
    vc = ops.Codec(c["D"], c["vb"], 1, rotation="dense")
    per_step = c["Hkv"] * int(lens.sum()) * (4 * kc.packed_width + 4 * vc.packed_width + 8)
    n_sets = max(2, math.ceil(args.rotate_mb * 1e6 / per_step))
    g = torch.Generator(device=dev).manual_seed(2000)
    sets = []
    for _ in range(n_sets):
        st = []
        for codec, x in zip((kc, vc), _synth_kv(torch, g, (c["B"], c["Hkv"], cap, c["D"]),
                                                  torch.bfloat16, dev)):
            pk = torch.empty((c["B"], c["Hkv"], cap, codec.packed_width), dtype=torch.uint32, device=dev)
            nm = torch.empty((c["B"], c["Hkv"], cap), dtype=torch.float32, device=dev)
            ops.append_quantize(x, codec, pk, nm, 0)
            st.append((nm, pk))
            del x
        sets.append(st)
        _free(torch)
    qs = [torch.randn(c["B"], c["Hq"], 1, c["D"], device=dev, generator=g).to(torch.bfloat16)
          for _ in range(n_sets)]
    lens_dev = torch.from_numpy(lens.astype(np.int32)).to(dev)
    scale = 1.0 / math.sqrt(c["D"])

    def step(i):
        (kn, kp), (vn, vp) = sets[i % n_sets]
        return ops.attention_packed(qs[i % n_sets], kn, kp, vn, vp, kc, vc, scale, False,
                                    seq_lens=lens_dev)

    steps = max(5, args.steps // 10)
    ms, outs, _ = graph_timed(torch, step, steps, max(2, args.warmup // 4), dev)
    if not torch.equal(outs[0], step(0)):
        raise RuntimeError("config 2: graph replay differs from the eager call")
    del sets, outs
    _free(torch)
    gbs = per_step / (ms * 1e-3) / 1e9
    return {"workload": "cfg2 ragged decode: 32 seqs, T~U[2048,8192] (seed 1004), 16 q / 8 kv heads, "
                        "d=256, K 4-bit / V 2-bit, dense 256x256 rotation, f32 norms, Beta codebooks",
            "value": round(gbs, 2), "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "us_per_step": round(ms * 1e3, 3), "sum_tokens": int(lens.sum()),
            "bytes_per_step": per_step, "decode_tokens_per_s": round(c["B"] * 1e3 / ms, 1),
            "steps": steps}


def bench_prefill_append(torch, args, dev):
    """Config 3: one 8192-token bf16 chunk appended to each of 36 layers.

    Layers 0-3 keep model-dtype K/V (plain copy); layers 4-35 rotate by a dense
    128x128 matrix on the matrix cores, quantize to 3 bits and pack.  Every
    layer reads its own input tensors, so nothing is served from cache.
    """
    from kaplumba_amd import ops

    c = CFG3
    H, T, D, bits = c["Hkv"], c["T"], c["D"], c["bits"]
    kc = ops.Codec(D, bits, 0, rotation="dense")
    vc = ops.Codec(D, bits, 1, rotation="dense")
    g = torch.Generator(device=dev).manual_seed(3000)
    inputs = [_synth_kv(torch, g, (1, H, T, D), torch.bfloat16, dev) for _ in range(c["layers"])]
    dst = []
    for li in range(c["layers"]):
        if li < c["plain_layers"]:
            dst.append([torch.empty((1, H, T, D), dtype=torch.bfloat16, device=dev) for _ in range(2)])
        else:
            dst.append([(torch.empty((1, H, T, codec.packed_width), dtype=torch.uint32, device=dev),
                         torch.empty((1, H, T), dtype=torch.float32, device=dev)) for codec in (kc, vc)])

    def layer(li):
        k, v = inputs[li]
        if li < c["plain_layers"]:
            ops.append_plain(k, dst[li][0], 0)
            ops.append_plain(v, dst[li][1], 0)
        else:
            (kp, kn), (vp, vn) = dst[li]
            ops.append_quantize_kv(k, v, kc, vc, kp, kn, vp, vn, 0)

    def step(_i):
        for li in range(c["layers"]):
            layer(li)

    n_q = c["layers"] - c["plain_layers"]

    def step_quant(_i):
        for li in range(c["plain_layers"], c["layers"]):
            layer(li)

    steps = max(3, args.steps // 40)
    ms, _, _ = graph_timed(torch, step, steps, 2, dev)
    ms_q, _, _ = graph_timed(torch, step_quant, steps, 2, dev)
    del inputs, dst
    _free(torch)
    qbytes = quantize_bytes(H * T, D, bits, 2, 4)           # one K or V launch
    pbytes = H * T * D * 2 * 2                              # plain layer tensor: read + write
    total = n_q * 2 * qbytes + c["plain_layers"] * 2 * pbytes
    launch_us = ms_q * 1e3 / (2 * n_q)                      # per K or V tensor (half a K+V launch)
    flops = 2.0 * H * T * D * D                             # u @ R^T per tensor
    return {"workload": "cfg3 prefill append: 36 layers x bf16 K,V [8,8192,128]; layers 0-3 stored "
                        "unquantized, 4-35 dense 128x128 rotation (matrix cores) + 3-bit pack, f32 norms, "
                        "Beta codebook",
            "value": round(total / (ms * 1e-3) / 1e9, 2), "unit": "GB/s",
            "frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_step": round(ms * 1e3, 2), "bytes_per_step": total,
            "prefill_tokens_per_s": round(T * 1e3 / ms, 1),
            "dense_quantize": {"us_per_tensor": round(launch_us, 3), "bytes_per_tensor": qbytes,
                               "launches": "one append_dense_kv_kernel per layer (K and V)",
                               "GB/s": round(qbytes / (launch_us * 1e-6) / 1e9, 2),
                               "rotation_tflops": round(flops / (launch_us * 1e-6) / 1e12, 1),
                               "mfma_frac": round(3 * flops / (launch_us * 1e-6) / 1e12
                                                  / MFMA_BF16_PEAK_TFLOPS, 4),
                               "note": "rotation_tflops counts u@R^T once; the matrix cores run it "
                                       "three times (bf16 pieces of R), which mfma_frac counts"},
            "steps": steps}


def bench_verify(torch, args, dev):
    """Config 4: batch 4 x 4 causal drafts over 131072 + 4 tokens, K2/V1, plus fp16 K/V."""
    from kaplumba_amd import ops

    c = CFG4
    B, H, T, D = c["B"], c["Hkv"], c["T"], c["D"]
    kc, vc = ops.Codec(D, c["kb"], 0), ops.Codec(D, c["vb"], 1)
    per_step = B * H * T * (4 * kc.packed_width + 4 * vc.packed_width + 8)
    n_sets = max(2, math.ceil(args.rotate_mb * 1e6 / per_step))
    g = torch.Generator(device=dev).manual_seed(4000)
    sets = []
    for _ in range(n_sets):
        st = []
        for codec, x in zip((kc, vc), _synth_kv(torch, g, (B, H, T, D), torch.float16, dev)):
            pk = torch.empty((B, H, T, codec.packed_width), dtype=torch.uint32, device=dev)
            nm = torch.empty((B, H, T), dtype=torch.float32, device=dev)
            ops.append_quantize(x, codec, pk, nm, 0)
            st.append((nm, pk))
            del x
        sets.append(st)
        _free(torch)
    qs = [torch.randn(B, c["Hq"], c["L"], D, device=dev, generator=g).to(torch.bfloat16)
          for _ in range(n_sets)]
    scale = 1.0 / math.sqrt(D)

    def step(i):
        (kn, kp), (vn, vp) = sets[i % n_sets]
        return ops.attention_packed(qs[i % n_sets], kn, kp, vn, vp, kc, vc, scale, True)

    steps = max(5, args.steps // 10)
    ms, outs, _ = graph_timed(torch, step, steps, max(2, args.warmup // 4), dev)
    if not torch.equal(outs[0], step(0)):
        raise RuntimeError("config 4: graph replay differs from the eager call")
    del sets, outs
    _free(torch)
    # fp16-layer variant: the same shape over unquantized K/V
    kv = _synth_kv(torch, g, (B, H, T, D), torch.float16, dev)
    plain_bytes = 2 * B * H * T * D * 2

    def step_plain(i):
        return ops.attention_plain(qs[i % n_sets], kv[0], kv[1], scale, True)

    steps_p = max(3, args.steps // 20)
    ms_p, _, _ = graph_timed(torch, step_plain, steps_p, 2, dev)
    del kv
    _free(torch)
    gbs = per_step / (ms * 1e-3) / 1e9
    gbs_p = plain_bytes / (ms_p * 1e-3) / 1e9
    return {"workload": "cfg4 verify: batch 4 x 4 causal drafts, 32 q / 8 kv heads, d=128, "
                        "131076 tokens, K 2-bit / V 1-bit, Hadamard rotation, f32 norms, Beta codebooks",
            "value": round(gbs, 2), "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "us_per_step": round(ms * 1e3, 3), "bytes_per_step": per_step,
            "verified_tokens_per_s": round(B * c["L"] * 1e3 / ms, 1), "steps": steps,
            "fp16_layer": {"value": round(gbs_p, 2), "unit": "GB/s",
                           "frac": round(gbs_p / HBM_PEAK_GBS, 4),
                           "us_per_step": round(ms_p * 1e3, 3), "bytes_per_step": plain_bytes,
                           "steps": steps_p}}


def bench_prefill_attention(torch, args, dev):
    """A 256-query causal prefill chunk over the packed cache (32 q / 8 kv heads, d=128, 3-bit).

    Roofline: matrix cores.  Algorithmic flops count the visible (causal)
    query-key pairs once for the scores and once for the value sum, 2 flops
    each per coordinate; the kernels run three f16 products per score
    (hi/lo split), which the figure does not credit.
    """
    from kaplumba_amd import ops

    c = CFGP
    B, Hq, H, L, T, D = c["B"], c["Hq"], c["Hkv"], c["L"], c["T"], c["D"]
    layers, kc, vc = make_layer_caches(torch, 4, c, dev)
    g = torch.Generator(device=dev).manual_seed(5000)
    qs = [torch.randn(B, Hq, L, D, device=dev, generator=g).to(torch.bfloat16) for _ in layers]
    scale = 1.0 / math.sqrt(D)

    def step(i):
        (kn, kp), (vn, vp) = layers[i % len(layers)]
        return ops.attention_packed(qs[i % len(qs)], kn, kp, vn, vp, kc, vc, scale, True)

    steps = max(5, args.steps // 10)
    ms, outs, _ = graph_timed(torch, step, steps, 3, dev)
    if not torch.equal(outs[0], step(0)):
        raise RuntimeError("prefill attention: graph replay differs from the eager call")
    del layers, outs
    _free(torch)
    visible = sum(T - L + i + 1 for i in range(L))  # keys seen by each query position
    flops = 4.0 * B * Hq * D * visible
    tflops = flops / (ms * 1e-3) / 1e12
    return {"workload": "prefill attention: one 256-query causal chunk ending an 8192-token "
                        "prompt, 32 q / 8 kv heads, d=128, 3-bit K/V, Hadamard rotation, f32 norms, "
                        "Beta codebook",
            "value": round(tflops, 2), "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "roofline": "mfma (f16/bf16 dense peak 2500 TFLOP/s)",
            "us_per_step": round(ms * 1e3, 3), "flops_per_step": flops,
            "cache_bytes": algorithmic_decode_bytes(H, T, D, c["bits"], c["bits"], 4, B),
            "prefill_tokens_per_s": round(L * 1e3 / ms, 1), "steps": steps}


def bench_prod_decode(torch, args, dev):
    """Config-1 decode with Prod-coded keys (3 bits: 2-bit MSE + one-bit QJL
    signs, the TurboQuant inner-product codec) and 3-bit MSE values."""
    from kaplumba_amd import ops
    from kaplumba_amd.prod import ProdCodec, attention_prod

    B, Hq, H, T, D = 1, CFG1["Hq"], CFG1["Hkv"], CFG1["T"], CFG1["D"]
    kc, vc = ProdCodec(D, 3, 0), ops.Codec(D, 3, 1)
    per_tok = 4 * kc.mse_width + 4 * kc.sign_width + 8 + 4 * vc.packed_width + 4
    per_step = B * H * T * per_tok
    n_sets = max(2, math.ceil(args.rotate_mb * 1e6 / per_step))
    g = torch.Generator(device=dev).manual_seed(6000)
    sets = []
    for _ in range(n_sets):
        k, v = _synth_kv(torch, g, (B, H, T, D), torch.float16, dev)
        kst = kc.alloc(B, H, T, dev)
        kc.quantize_into(k, kst, 0)
        vp = torch.empty((B, H, T, vc.packed_width), dtype=torch.uint32, device=dev)
        vn = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        ops.append_quantize(v, vc, vp, vn, 0)
        sets.append((kst, vn, vp))
        del k, v
    _free(torch)
    qs = [torch.randn(B, Hq, 1, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(n_sets)]
    scale = 1.0 / math.sqrt(D)

    def step(i):
        kst, vn, vp = sets[i % n_sets]
        return attention_prod(qs[i % n_sets], kst, vn, vp, kc, vc, scale, False)

    steps = max(5, args.steps // 4)
    ms, outs, _ = graph_timed(torch, step, steps, max(2, args.warmup // 4), dev)
    if not torch.equal(outs[0], step(0)):
        raise RuntimeError("Prod decode: graph replay differs from the eager call")
    del sets, outs
    _free(torch)
    gbs = per_step / (ms * 1e-3) / 1e9
    return {"workload": "cfg1 decode with Prod keys: 3-bit Prod K (2-bit MSE + 1-bit QJL signs, "
                        "f32 norm and residual norm) and 3-bit MSE V, 32 q / 8 kv heads, d=128, "
                        "32768 tokens, Beta codebooks",
            "value": round(gbs, 2), "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "us_per_step": round(ms * 1e3, 3), "bytes_per_step": per_step,
            "note": "one call = qprep_kernel (q @ P^T) + attn_small_kernel (Prod) + attn_merge_kernel",
            "steps": steps}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sample, seconds_budget=12.0):
    """The reference's array-path attention (oracle restatements) on the host.

    ``sample`` is the first layer cache of the headline leg copied to host
    memory (the append kernel's bytes, which equal the oracle quantizer's), so
    the CPU works on exactly the cfg1 workload: 8 kv heads x 32768 tokens.
    The torch-CPU restatement runs on all the threads torch is given (the
    figure reported); the numpy restatement runs once, single-threaded, beside it.
    """
    import numpy as np
    import torch

    from oracle import tq_oracle as O
    from oracle import tq_oracle_torch as OT

    c = CFG1
    q, kp, kn, vp, vn = sample
    T = kp.shape[2]
    cb = O.beta_codebook(c["D"], c["bits"])
    kw = dict(k_bits=c["bits"], v_bits=c["bits"], k_codebook=cb, v_codebook=cb,
              signs_k=O.rht_signs(c["D"], 0), signs_v=O.rht_signs(c["D"], 1),
              scale=1 / math.sqrt(c["D"]), q_dtype="bf16")
    threads = torch.get_num_threads()
    runs = []
    t_start = time.perf_counter()
    while len(runs) < 3 or (time.perf_counter() - t_start < seconds_budget and len(runs) < 30):
        t0 = time.perf_counter()
        OT.attention_chunked(q, kp, kn, vp, vn, key_chunk=1 << 30, **kw)
        runs.append(time.perf_counter() - t0)
    med = sorted(runs)[len(runs) // 2]
    t0 = time.perf_counter()
    O.attention_chunked_f32(q, kp, kn, vp, vn, key_chunk=1 << 30, **kw)
    t_np = time.perf_counter() - t0
    nbytes = algorithmic_decode_bytes(c["Hkv"], T, c["D"], c["bits"], c["bits"], 4)
    return {"value": round(nbytes / med / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu": _cpu_model(), "host_cores_visible": len(os.sched_getaffinity(0)),
            "torch_threads": threads, "ms_per_step": round(med * 1e3, 2),
            "numpy_single_thread": {"value": round(nbytes / t_np / 1e9, 4), "unit": "GB/s",
                                    "ms_per_step": round(t_np * 1e3, 1)},
            "sample": f"the cfg1 workload itself: one layer cache (8 kv heads x {T} tokens, 3-bit, "
                      f"f32 norms) and its bf16 query, attention by the torch-CPU restatement of the "
                      f"reference array path (oracle/tq_oracle_torch.py) on {threads} threads, median "
                      f"of {len(runs)} runs; reference algorithm, torch/numpy restatement -- not MLX"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rotate-mb", type=float, default=600.0,
                    help="total size of distinct caches walked by successive steps")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--tokens", type=int, default=CFG1["T"],
                    help="cached tokens per kv head of the headline decode leg (context-length "
                         "sweeps; the config-1 figure is quoted at the default 32768)")
    ap.add_argument("--legs", default="cfg0,cfg2,cfg3,cfg4,prefill,prod",
                    help="comma-separated extra legs to run after the cfg1 headline "
                         "(cfg0, cfg2, cfg3, cfg4, prefill, prod; empty for the headline only)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode shards by kv head or by context; see DESIGN.md).", file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda", 0)
    dec = bench_decode(torch, args, dev)
    _free(torch)
    floor = bench_floor(torch, dev, dec["bytes"], dec["n_layers"])
    legs = {x.strip() for x in args.legs.split(",") if x.strip()}
    unknown = legs - {"cfg0", "cfg2", "cfg3", "cfg4", "prefill", "prod"}
    if unknown:
        ap.error(f"unknown legs: {sorted(unknown)}")
    value = dec["bytes"] / (dec["ms_per_step"] * 1e-3) / 1e9
    line = {
        "metric": "packed-KV decode attention GB/s (% HBM peak) @32k ctx 3-bit; quantize GB/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (3-bit packed K/V, bf16 q/out)",
        "data": "synthetic",
        "config": {"workload": "cfg1 decode attention, 3-bit TurboQuant KV, batch 1, 32 q heads / "
                               "8 kv heads, d=128, 32768 tokens, Hadamard rotation, f32 norms, "
                               "Beta Lloyd-Max codebook (the reference's live _codebook)",
                   "codebook_note": CODEBOOK_NOTE,
                   "tokens": args.tokens, "bytes_per_step": dec["bytes"],
                   "distinct_layer_caches": dec["n_layers"], "rotated_mb": round(dec["rotate_mb"], 1),
                   "decode_tokens_per_s": round(1e3 / dec["ms_per_step"], 1),
                   "timing": "HIP graph of the timed steps, one replay bracketed by HIP events"},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": CFG1_TRAFFIC_BYTES,
                     "traffic_note": "HBM bytes per call from rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                                     "copy-calibrated; algorithmic bytes are 27,262,976",
                     "frac_of_copy_peak": round(value / floor["stream_read"]["GB/s"], 4),
                     "frac_of_device_copy": round(value / floor["device_copy"]["GB/s"], 4),
                     "copy_peak": floor,
                     "copy_peak_note": "frac_of_copy_peak = achieved / the stream-read probe moving "
                                       "the same bytes per launch over the same number of distinct "
                                       "buffers (the floor of one call); frac_of_device_copy = "
                                       "achieved / a 1 GiB device copy",
                     "kernel": "attention call: attn_stage_kernel<128,3,3> + attn_merge_rot_kernel<128>",
                     "call_us": round(dec["ms_per_step"] * 1e3, 3),
                     "achieved_note": "algorithmic bytes / time of one whole attention call (both "
                                      "kernels, HIP events around a graph replay); the per-kernel "
                                      "durations are in the committed rocprofv3 summaries"},
    }
    if "cfg0" in legs:
        qnt = bench_quantize(torch, args, dev)
        _free(torch)
        line["quantize"] = {"workload": "cfg0 append-quantize K+V f16 [1,8,4096,128] 3-bit (one "
                                        "tq_append_quantize_kv call, as update_and_fetch makes), "
                                        "Hadamard rotation, Beta codebook",
                            "value": round(qnt["bytes"] / (qnt["ms_per_step"] * 1e-3) / 1e9, 2),
                            "unit": "GB/s", "step_us": round(qnt["ms_per_step"] * 1e3, 3)}
    if "cfg2" in legs:
        line["cfg2"] = bench_ragged(torch, args, dev)
    if "cfg3" in legs:
        line["cfg3"] = bench_prefill_append(torch, args, dev)
    if "cfg4" in legs:
        line["cfg4"] = bench_verify(torch, args, dev)
    if "prefill" in legs:
        line["prefill_attention"] = bench_prefill_attention(torch, args, dev)
    if "prod" in legs:
        line["prod_decode"] = bench_prod_decode(torch, args, dev)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(dec["cpu_sample"])
    print(json.dumps(line))


if __name__ == "__main__":
    main()
