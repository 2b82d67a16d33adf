"""GPU parity of decode / verify attention (C ABI tq_attention) vs the oracle.

Bar: outputs within 2e-3 max-abs and 1e-3 mean-rel of
the float64 TurboQuant attention.  Both sides are rounded to the query dtype,
as the reference casts its f32 result (``.astype(queries.dtype)``); a bf16
output cannot resolve differences below its own ulp (3.9e-3 for values in
[0.5, 1)), so an element passes when |got - want| <= max(2e-3, ulp(want)).
mean-rel is mean(|got - want|) / mean(|want|) <= 1e-3.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from kaplumba_amd import ops

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_REL = 1e-3
QDT = {0: "f32", 1: "f16", 2: "bf16"}
TORCH_QDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


MANT_BITS = {"f32": 23, "f16": 10, "bf16": 7}
# every assert_close call's margins; conftest writes them out when
# TQ_MARGINS_OUT names a file
MARGINS = []


def dtype_ulp(w: np.ndarray, qdt: str) -> np.ndarray:
    """Spacing of the query dtype at |w| (normal range)."""
    a = np.maximum(np.abs(w), 1e-30)
    return np.exp2(np.floor(np.log2(a)) - MANT_BITS[qdt])


def assert_close(got: torch.Tensor, want64: np.ndarray, qdt: str, label=""):
    g = got.float().cpu().numpy().astype(np.float64)
    w = O.round_to_dtype(want64.astype(np.float32), qdt).astype(np.float64)
    err = np.abs(g - w)
    tol = np.maximum(MAX_ABS, dtype_ulp(w, qdt))
    mean_rel = err.mean() / max(np.abs(w).mean(), 1e-30)
    n_ulp = int((err > MAX_ABS).sum())
    print(f"[{label}] max_abs={err.max():.3e} mean_rel={mean_rel:.3e} one-ulp-flips>2e-3: {n_ulp}",
          flush=True)
    MARGINS.append({"label": label, "max_abs": float(err.max()), "mean_rel": float(mean_rel),
                    "elements": int(err.size), "over_2e-3_within_one_ulp": n_ulp})
    assert (err <= tol).all(), (label, err.max(), float((err - tol).max()))
    assert mean_rel <= MEAN_REL, (label, mean_rel)


def to_buffers(kp, kn, vp, vn, device, extra=7, norm_dtype=torch.float32):
    """Place (B, H, T, PW)/(B, H, T) arrays in larger capacity buffers; return views."""
    B, H, T = kn.shape
    cap = T + extra
    out = []
    for p, n in ((kp, kn), (vp, vn)):
        pb = torch.zeros((B, H, cap, p.shape[-1]), dtype=torch.uint32, device=device)
        nb = torch.zeros((B, H, cap), dtype=norm_dtype, device=device)
        pb[:, :, :T] = torch.from_numpy(p.astype(np.uint32)).to(device)
        nb[:, :, :T] = torch.from_numpy(np.asarray(n, np.float32)).to(device).to(norm_dtype)
        out += [nb[:, :, :T], pb[:, :, :T]]
    return out  # k_norms, k_idx, v_norms, v_idx


def q_tensor(q_np, qdt, device):
    return torch.from_numpy(q_np.astype(np.float32)).to(TORCH_QDT[qdt]).to(device)


@pytest.mark.parametrize("case", ["decode_d128_k3v3", "verify_d128_k2v1", "ragged_d256_k4v2_dense",
                                  "decode_d64_k4v4_f32q"])
def test_golden_cases(golden, device, case):
    a = golden["attention"]
    B, Hq, Hkv, L, T, d, kb, vb, dense, causal = (int(v) for v in a[f"{case}/meta"])
    qdt = QDT[int(a[f"{case}/qdtype"][0])]
    rot = "dense" if dense else "hadamard"
    kn, ki, vn, vi = to_buffers(a[f"{case}/k_packed"], a[f"{case}/k_norms"], a[f"{case}/v_packed"],
                                a[f"{case}/v_norms"], device)
    kc, vc = ops.Codec(d, kb, 0, rot), ops.Codec(d, vb, 1, rot)
    lengths = torch.from_numpy(a[f"{case}/lengths"]).to(device)
    out = ops.attention_packed(q_tensor(a[f"{case}/q"], qdt, device), kn, ki, vn, vi, kc, vc,
                               1.0 / math.sqrt(d), bool(causal), seq_lens=lengths)
    assert_close(out, a[f"{case}/expected"].astype(np.float64), qdt, case)


def test_golden_plain_f16(golden, device):
    a = golden["attention"]
    q = q_tensor(a["plain_f16/q"], "f16", device)
    kb = torch.zeros((1, 2, 230, 128), dtype=torch.float16, device=device)
    vb = torch.zeros_like(kb)
    kb[:, :, :200] = torch.from_numpy(a["plain_f16/k"]).to(device)
    vb[:, :, :200] = torch.from_numpy(a["plain_f16/v"]).to(device)
    out = ops.attention_plain(q, kb[:, :, :200], vb[:, :, :200], 1 / math.sqrt(128), True)
    assert_close(out, a["plain_f16/expected"].astype(np.float64), "f16", "plain_f16")


def build_case(seed, B, Hq, Hkv, L, T, d, kb, vb, rot="hadamard", qdt="bf16", norm="float32"):
    rng = np.random.default_rng(seed)
    s = np.exp(rng.normal(0, 0.5, size=(1, Hkv, 1, d)))
    k = (rng.standard_normal((B, Hkv, T, d)) * s).astype(np.float16).astype(np.float32)
    v = (rng.standard_normal((B, Hkv, T, d)) * s).astype(np.float16).astype(np.float32)
    if rot == "hadamard":
        kr, vr = O.rht_signs(d, 0), O.rht_signs(d, 1)
        kp, kn = O.quantize_rht(k, kb, kr, O.beta_codebook(d, kb), norm)
        vp, vn = O.quantize_rht(v, vb, vr, O.beta_codebook(d, vb), norm)
    else:
        kr, vr = O.rotation_matrix(d, 0), O.rotation_matrix(d, 1)
        kp, kn, _ = O.quantize_dense(k, kb, kr, O.beta_codebook(d, kb), norm)
        vp, vn, _ = O.quantize_dense(v, vb, vr, O.beta_codebook(d, vb), norm)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), qdt)
    return q, kp, kn, vp, vn, kr, vr


def run_case(device, seed, B, Hq, Hkv, L, T, d, kb, vb, rot="hadamard", qdt="bf16", causal=None,
             lengths=None, norm="float32", starts=None, v_codebook=None):
    """v_codebook: value levels to attend with in place of the Beta codebook
    (the cache's indices are drawn with the Beta codebook either way)."""
    causal = (L > 1) if causal is None else causal
    q, kp, kn, vp, vn, kr, vr = build_case(seed, B, Hq, Hkv, L, T, d, kb, vb, rot, qdt, norm)
    vcb = O.beta_codebook(d, vb) if v_codebook is None else np.asarray(v_codebook, np.float32)
    want = O.attention(q, kp, kn, vp, vn, k_bits=kb, v_bits=vb, k_codebook=O.beta_codebook(d, kb),
                       v_codebook=vcb, rot_kind=rot, k_rot=kr, v_rot=vr,
                       scale=1 / math.sqrt(d), q_dtype=qdt, causal=causal, lengths=lengths,
                       starts=starts)
    nd = torch.float16 if norm == "float16" else torch.float32
    kn_t, ki, vn_t, vi = to_buffers(kp, kn, vp, vn, device, norm_dtype=nd)
    sl = torch.tensor(lengths, dtype=torch.int32, device=device) if lengths is not None else None
    vcodec = ops.Codec(d, vb, 1, rot)
    if v_codebook is not None:
        vcodec.codebook = vcb
        vcodec.midpoints = O.midpoints(vcb)
    out = ops.attention_packed(q_tensor(q, qdt, device), kn_t, ki, vn_t, vi,
                               ops.Codec(d, kb, 0, rot), vcodec,
                               1 / math.sqrt(d), causal, seq_lens=sl,
                               seq_starts=None if starts is None else torch.tensor(starts))
    label = f"B{B} Hq{Hq} Hkv{Hkv} L{L} T{T} d{d} k{kb}v{vb} {rot} {qdt}"
    if starts is not None:
        label += f" starts{list(starts)}"
    assert_close(out, want, qdt, label)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kb,vb", [(1, 1), (2, 2), (3, 3), (4, 4), (4, 2), (2, 1), (3, 4), (1, 3)])
def test_decode_bits_and_dims(device, d, kb, vb):
    run_case(device, 100 + d + 10 * kb + vb, 1, 8, 2, 1, 777, d, kb, vb)


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (8, 1), (24, 8)])
@pytest.mark.parametrize("L", [1, 2, 4])
def test_gqa_groups_and_verify_rows(device, Hq, Hkv, L):
    run_case(device, Hq * 7 + Hkv + L, 1, Hq, Hkv, L, 1500, 128, 3, 3)


@pytest.mark.parametrize("Hq,Hkv,L,d,kb,vb,rot", [
    (16, 8, 1, 256, 4, 2, "dense"),     # d = 256, 4-row groups, dense rotation
    (8, 4, 2, 256, 2, 3, "hadamard"),   # d = 256, causal verify rows
    (32, 2, 1, 64, 3, 3, "hadamard"),   # 16-row groups at d = 64
])
@pytest.mark.parametrize("shape", ["extreme", "tiny"])
def test_ragged_lengths_general_kernel(device, Hq, Hkv, L, d, kb, vb, rot, shape):
    # The general kernel over very uneven sequence lengths: empty sequences
    # (zero rows), sequences shorter than one 32-token sub-chunk, lengths on
    # and next to sub-chunk and split boundaries, and (tiny) a batch whose
    # whole cache is a few tokens.
    if shape == "extreme":
        lens = [0, 1, 31, 32, 33, 3000, 17, 2999, 64, 1500, 0, 2048]
        T = 3000
    else:
        lens = [1, 0, 2, 3, 1, 0, 2, 1]
        T = 3
    run_case(device, 11 + d + L, len(lens), Hq, Hkv, L, T, d, kb, vb, rot=rot, lengths=lens)


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 2048, 5000])
def test_token_counts(device, T):
    run_case(device, T, 1, 8, 2, 1, T, 128, 3, 3)
    run_case(device, T + 1, 1, 8, 2, 4, max(T, 4), 128, 2, 1)


@pytest.mark.parametrize("qdt", ["f32", "f16", "bf16"])
def test_query_dtypes_and_f16_norms(device, qdt):
    run_case(device, 5, 2, 8, 2, 1, 600, 128, 3, 3, qdt=qdt, norm="float16")


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 1), (1, 2), (2, 2)])
@pytest.mark.parametrize("Hq,Hkv,L,T,qdt,norm", [
    (16, 8, 1, 2500, "bf16", "float32"),   # two rows per kv head, several splits
    (8, 2, 1, 300, "f32", "float16"),      # four rows, one split (finished in the kernel)
    (4, 2, 2, 1234, "f16", "float32"),     # two causal verify rows per head
])
def test_d256_dense_row_groups(device, kb, vb, Hq, Hkv, L, T, qdt, norm):
    """d = 256, dense rotation, <= 4 rows per kv head and 1- or 2-bit values: the staged
    row-group kernel, for every key width."""
    run_case(device, 300 + 10 * kb + vb + L, 2, Hq, Hkv, L, T, 256, kb, vb, rot="dense",
             qdt=qdt, norm=norm)


def test_ragged_batch_dense_d256(device):
    """Config-2 shape at reduced size: ragged lengths, d=256, K4/V2, dense rotation."""
    lengths = [300, 1, 1700, 0, 999]
    run_case(device, 77, 5, 16, 8, 1, 1700, 256, 4, 2, rot="dense", lengths=lengths)


@pytest.mark.parametrize("d,Hq,Hkv,L,T", [
    (64, 8, 2, 1, 3000),     # 4-row groups, many splits
    (128, 32, 8, 4, 2500),   # 16-row groups (GQA 4 x 4 drafts), causal
    (128, 8, 8, 1, 700),     # MHA, one row per group
    (256, 8, 2, 3, 2100),    # three 4-row groups per kv head, causal
    (128, 32, 8, 32, 300),   # 2,048 query rows: the query rotation's 16-row blocks
])
def test_dense_rotation_shapes(device, d, Hq, Hkv, L, T):
    """Dense R_K / R_V: the query rotation and the merge's R_V^-1 over whole row groups."""
    run_case(device, 40 + d + L, 2, Hq, Hkv, L, T, d, 3, 2, rot="dense")


def test_ragged_verify_causal(device):
    run_case(device, 78, 3, 8, 2, 4, 900, 128, 2, 1, lengths=[4, 900, 517], causal=True)


def test_ragged_verify_small_row_groups(device):
    """Ragged causal verify with 4 query rows per kv head (GQA 2 x 2 drafts)."""
    run_case(device, 79, 3, 4, 2, 2, 2600, 128, 3, 3, lengths=[4, 2600, 517], causal=True)


@pytest.mark.parametrize("d", [64, 128])
def test_split_with_fully_masked_rows(device, d):
    """T = 9 * 256 + 2 with 4 causal drafts: the last split holds 2 keys that rows 0 and 1
    may not see, so those rows' partials carry only masked scores."""
    run_case(device, 80 + d, 1, 2, 2, 4, 9 * 256 + 2, d, 3, 3, causal=True)


@pytest.mark.parametrize("Hq,Hkv,L,kb,vb,lengths", [
    (32, 8, 4, 2, 1, None),            # config-4 shape: 16 rows (GQA 4 x 4 drafts), causal
    (16, 8, 3, 3, 3, None),            # 6 rows: the idle columns of the group
    (32, 2, 1, 4, 4, None),            # GQA-16 decode
    (8, 1, 2, 1, 3, None),             # 8 heads x 2 drafts
    (32, 8, 4, 3, 2, [5000, 3, 777]),  # ragged, one sequence shorter than the drafts
    (4, 1, 40, 3, 3, None),            # 160 rows: ten row groups (a prefill chunk)
    (24, 8, 4, 2, 2, [1, 4100]),       # 12 rows, ragged with a one-token sequence
    (16, 4, 4, 1, 1, [4999, 2600]),    # 1-bit keys and values, ragged
])
def test_rows16_groups(device, Hq, Hkv, L, kb, vb, lengths):
    """16-row groups at d = 128 (verify, wide GQA, prefill chunks)."""
    B = 1 if lengths is None else len(lengths)
    T = 5000 if lengths is None else max(lengths)
    run_case(device, 300 + Hq + L + kb, B, Hq, Hkv, L, T, 128, kb, vb, lengths=lengths)


@pytest.mark.parametrize("qdt", ["f32", "f16"])
@pytest.mark.parametrize("kb,vb", [(3, 3), (2, 1)])
def test_rows16_query_dtypes_and_f16_norms(device, qdt, kb, vb):
    run_case(device, 6, 2, 32, 8, 2, 1300, 128, kb, vb, qdt=qdt, norm="float16")


@pytest.mark.parametrize("Hq,Hkv,L,kb,vb,T", [
    (32, 8, 4, 2, 1, 5000),   # 16-row groups (verify)
    (32, 8, 4, 1, 1, 777),    # 16-row groups, one split
    (8, 2, 1, 2, 1, 3000),    # <= 4 rows per kv head (decode)
    (8, 1, 16, 3, 1, 2100),   # 128 rows: prefill tiles
])
def test_asymmetric_one_bit_value_codebook(device, Hq, Hkv, L, kb, vb, T):
    """A 1-bit value codebook whose levels are not symmetric about zero: the
    16-row kernel forms v = mid + half * s with s = +-1, so the midpoint term
    (the sum of the weights) must be carried; the other kernels read the
    levels directly."""
    run_case(device, 70 + L + kb, 1, Hq, Hkv, L, T, 128, kb, vb, v_codebook=[-0.031, 0.094])


def test_rows16_split_with_fully_masked_rows(device):
    """16 causal drafts over T = 9 * 256 + 2: in the last split most rows see
    no key, so their partials carry only masked scores."""
    run_case(device, 81, 1, 1, 1, 16, 9 * 256 + 2, 128, 3, 3, causal=True)


@pytest.mark.parametrize("d,Hq,Hkv,L", [(128, 8, 2, 1), (64, 4, 2, 2), (128, 32, 8, 2), (256, 8, 2, 1)])
def test_f16_norms_odd_sequence_ends(device, d, Hq, Hkv, L):
    """f16 norms (the reference layout) with odd sequence ends: the last
    token's norm shares a dword with the position past the end, which a
    bounded 16-byte load reads as zero; the kernels must still use it."""
    run_case(device, 90 + d + Hq + L, 3, Hq, Hkv, L, 701, d, 3, 3, qdt="f16", norm="float16",
             lengths=[5, 701, 33])


def test_empty_cache_gives_zeros(device):
    q = torch.randn(1, 8, 1, 128, dtype=torch.bfloat16, device=device)
    kc, vc = ops.Codec(128, 3, 0), ops.Codec(128, 3, 1)
    kn = torch.zeros((1, 2, 4), device=device)
    ki = torch.zeros((1, 2, 4, 12), dtype=torch.uint32, device=device)
    out = ops.attention_packed(q, kn[:, :, :0], ki[:, :, :0], kn[:, :, :0], ki[:, :, :0], kc, vc,
                               0.1, False)
    assert out.shape == (1, 8, 1, 128) and not out.float().abs().sum().item()


def test_repeated_calls_reuse_workspace(device):
    """One cached workspace serves calls of different group and split counts in turn."""
    for B, Hkv, T in ((1, 2, 300), (3, 8, 5000), (1, 2, 300), (2, 4, 70)):
        run_case(device, B * 13 + T, B, Hkv * 4, Hkv, 1, T, 128, 3, 3)


def test_graph_survives_a_larger_workspace(device):
    """A graph captured on a stream keeps its workspace address.  A later,
    larger call on that stream moves the stream to a new workspace; the old
    one must stay allocated, so replaying the graph still gives its eager
    output (and a tensor allocated meanwhile is not overwritten)."""
    kc, vc = ops.Codec(128, 3, 0), ops.Codec(128, 3, 1)

    def problem(seed, B, Hkv, T):
        q, kp, kn, vp, vn, _, _ = build_case(seed, B, 4 * Hkv, Hkv, 1, T, 128, 3, 3)
        return q_tensor(q, "bf16", device), to_buffers(kp, kn, vp, vn, device)

    s = torch.cuda.Stream(device=device)
    s.wait_stream(torch.cuda.current_stream(device))
    small_q, small_kv = problem(1, 1, 2, 700)
    big_q, big_kv = problem(2, 4, 8, 20000)
    with torch.cuda.stream(s):
        call = lambda q, kv: ops.attention_packed(q, kv[0], kv[1], kv[2], kv[3], kc, vc, 0.088, False)
        eager = call(small_q, small_kv)  # workspace sized for the small problem
        torch.cuda.synchronize(device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            captured = call(small_q, small_kv)
        big = call(big_q, big_kv)        # needs a larger workspace on this stream
        guard = torch.full((1 << 22,), 3.0, device=device)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize(device)
            assert torch.equal(captured, eager)
            assert bool((guard == 3.0).all())
    torch.cuda.synchronize(device)
    assert torch.equal(call(big_q, big_kv), big)


@pytest.mark.parametrize("codebook", ["beta", "gaussian"])
def test_config1_full_size(device, codebook):
    """Config 1: 32 q heads / 8 kv heads, d=128, 32768 tokens, 3-bit, bf16 query.

    The cache is written by the HIP append kernel (bit-exact vs the oracle)
    and attention is checked against the float64 oracle at full size, with
    the reference's Beta codebook and with BASELINE's N(0,1) Lloyd-Max one.
    """
    rs, rk, rv, rq = (np.random.default_rng(s) for s in (1000, 1001, 1002, 1003))
    T = 32768
    scale = np.exp(rs.normal(0.0, 0.5, size=(1, 8, 1, 128)))
    k = (rk.standard_normal((1, 8, T, 128)) * scale).astype(np.float16)
    v = (rv.standard_normal((1, 8, T, 128)) * scale).astype(np.float16)
    q = O.round_to_dtype(rq.standard_normal((1, 32, 1, 128)).astype(np.float32), "bf16")
    kc = ops.Codec(128, 3, 0, codebook_kind=codebook)
    vc = ops.Codec(128, 3, 1, codebook_kind=codebook)
    cb = O.beta_codebook(128, 3) if codebook == "beta" else O.gaussian_codebook(128, 3)
    bufs = []
    for x, c in ((k, kc), (v, vc)):
        pb = torch.zeros((1, 8, T, 12), dtype=torch.uint32, device=device)
        nb = torch.zeros((1, 8, T), dtype=torch.float32, device=device)
        ops.append_quantize(torch.from_numpy(x).to(device), c, pb, nb, 0)
        bufs.append((pb, nb))
    (kp, kn), (vp, vn) = bufs
    kp_np, vp_np = kp.cpu().numpy().astype(np.uint32), vp.cpu().numpy().astype(np.uint32)
    wkp, wkn = O.quantize_rht(k, 3, O.rht_signs(128, 0), cb)
    assert np.array_equal(kp_np, wkp) and np.array_equal(kn.cpu().numpy(), wkn)
    out = ops.attention_packed(q_tensor(q, "bf16", device), kn, kp, vn, vp, kc, vc,
                               1 / math.sqrt(128), False)
    want = O.attention(q, kp_np, kn.cpu().numpy(), vp_np, vn.cpu().numpy(), k_bits=3, v_bits=3,
                       k_codebook=cb, v_codebook=cb,
                       rot_kind="hadamard", k_rot=O.rht_signs(128, 0), v_rot=O.rht_signs(128, 1),
                       scale=1 / math.sqrt(128), q_dtype="bf16")
    assert_close(out, want, "bf16", f"config1 full size, {codebook} codebook")


@pytest.mark.parametrize("kvdt", ["f16", "bf16"])
@pytest.mark.parametrize("d,Hq,Hkv,L,T,lengths", [
    (128, 32, 8, 4, 5000, None),        # cfg4 shape at reduced length: 16-row groups, causal
    (128, 8, 8, 1, 3000, None),         # MHA decode, 4-row groups, many splits
    (64, 16, 2, 1, 2600, [2600, 17]),   # ragged, 16-row groups (GQA 8 x 2 rows)
    (256, 16, 8, 3, 2300, [900, 2300]), # d=256 verify, ragged
    (128, 4, 1, 1, 200, None),          # one split: finished inside the partial kernel
])
def test_plain_layers(device, kvdt, d, Hq, Hkv, L, T, lengths):
    """fp16 / bf16 layers (the mixed-precision split) through the matrix-core plain kernel."""
    rng = np.random.default_rng(d + L + T)
    B = 2 if lengths is not None else 1
    tdt = TORCH_QDT[kvdt]
    s = np.exp(rng.normal(0, 0.5, size=(1, Hkv, 1, d)))
    k = torch.from_numpy((rng.standard_normal((B, Hkv, T, d)) * s).astype(np.float32)).to(tdt)
    v = torch.from_numpy((rng.standard_normal((B, Hkv, T, d)) * s).astype(np.float32)).to(tdt)
    q = O.round_to_dtype(rng.standard_normal((B, Hq, L, d)).astype(np.float32), "bf16")
    causal = L > 1
    want = O.attention_plain(q, k.float().numpy(), v.float().numpy(), scale=1 / math.sqrt(d),
                             q_dtype="bf16", causal=causal, lengths=lengths)
    cap = T + 9
    kb = torch.zeros((B, Hkv, cap, d), dtype=tdt, device=device)
    vb = torch.zeros_like(kb)
    kb[:, :, :T] = k.to(device)
    vb[:, :, :T] = v.to(device)
    sl = torch.tensor(lengths, dtype=torch.int32, device=device) if lengths is not None else None
    out = ops.attention_plain(q_tensor(q, "bf16", device), kb[:, :, :T], vb[:, :, :T],
                              1 / math.sqrt(d), causal, seq_lens=sl)
    assert_close(out, want, "bf16", f"plain {kvdt} d{d} Hq{Hq} Hkv{Hkv} L{L} T{T}")


@pytest.mark.parametrize("Hq,Hkv,L,kb,vb,rot,lengths,starts,qdt,norm", [
    (8, 1, 9, 3, 3, "hadamard", None, None, "bf16", "float32"),          # 72 rows: one partial block
    (32, 8, 25, 4, 2, "hadamard", [3000, 17], None, "bf16", "float32"),  # 100 rows, ragged (one short)
    (16, 4, 50, 2, 1, "dense", None, None, "f16", "float16"),            # 200 rows: full + partial block
    (4, 1, 64, 1, 4, "hadamard", [1500, 1500], [0, 700], "bf16", "float32"),  # left padding
    (8, 2, 32, 4, 4, "hadamard", [33, 2000], None, "f32", "float32"),    # 128 rows, a 33-token sequence
    (2, 1, 80, 3, 3, "hadamard", None, None, "bf16", "float16"),         # L > T - causal rows see nothing
    (8, 2, 32, 3, 2, "hadamard", [0, 1, 2600], None, "bf16", "float32"), # empty and 1-token sequences
    (8, 2, 16, 2, 2, "dense", [700, 0], [300, 0], "f16", "float32"),     # left padding + an empty row
])
def test_tile_rows(device, Hq, Hkv, L, kb, vb, rot, lengths, starts, qdt, norm):
    """64 or more query rows per kv head at d = 128: the tile kernel (K/V decoded
    into LDS once per 32-token sub-chunk and shared by 128 rows)."""
    B = 1 if lengths is None else len(lengths)
    T = 1100 if lengths is None else max(lengths)
    if L == 80:
        T = 60  # more queries than keys: the first rows see no key (uniform weights)
    run_case(device, 900 + L + kb, B, Hq, Hkv, L, T, 128, kb, vb, rot=rot, qdt=qdt, norm=norm,
             lengths=lengths, starts=starts)
