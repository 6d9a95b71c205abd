"""GPU parity of the decode-step glue: RMSNorm and decode attention (RoPE,
float16 KV-cache append, GQA softmax attention) against the oracle's
restatement of the reference (oracle/decode_ref.py).

Tolerances: RMSNorm float32 output within 2e-6 relative of the fp64 form
(two correctly rounded float32 operations after a float32 sum of squares);
its bfloat16 output is the round-to-nearest-even of the float32 one.  The
appended float16 key is within one float16 ulp of the fp64 rotation of the
reference's float32 RoPE angles; the attention output meets the matmul bar
(max elementwise relative error 1e-3, floor 1e-3 * max) against the fp64
closed form over the cache contents."""

import numpy as np
import pytest
import torch

from dracort_amd.kernels import DecodeAttentionWorkspace, decode_attention, rms_norm, rope_tables
from oracle import decode_ref
from tests.gguf_cases import check_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n", [(1, 4096), (3, 4096), (16, 14336), (2, 8)])
def test_rms_norm(m, n):
    rng = np.random.default_rng(m * n)
    x = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    x[0, :5] = [40.0, -1e-3, 0.0, 7.5, -12.0]
    w = rng.standard_normal(n).astype(np.float32)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    yb = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    print(f"rms_norm [{m},{n}]", flush=True)
    y = rms_norm(xd, wd, 1e-5, out=torch.empty((m, n), device="cuda"), out_bf16=yb).cpu().numpy()
    ref = decode_ref.rms_norm_f64(x, w, 1e-5)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-30)) < 2e-6
    assert torch.equal(yb.cpu(), torch.from_numpy(y).to(torch.bfloat16))
    assert np.max(np.abs(y - decode_ref.rms_norm(x, w, 1e-5)) / np.maximum(np.abs(ref), 1e-30)) < 2e-6


def _attention_case(b, hq, hkv, d, max_pos, positions, theta, rope, seed, out_dtype=torch.float32):
    rng = np.random.default_rng(seed)
    kc = rng.standard_normal((b, hkv, max_pos, d)).astype(np.float16)
    vc = rng.standard_normal((b, hkv, max_pos, d)).astype(np.float16)
    q = rng.standard_normal((b, hq * d)).astype(np.float32)
    k = rng.standard_normal((b, hkv * d)).astype(np.float32)
    v = rng.standard_normal((b, hkv * d)).astype(np.float32)
    kcd, vcd = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    pos = torch.tensor(positions, dtype=torch.int32, device="cuda")
    tables = rope_tables(d, max_pos, theta) if rope else None
    out = decode_attention(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                           kcd, vcd, pos, hq, hkv, rope=tables, out_dtype=out_dtype)
    got = out.float().cpu().numpy()
    kc_gpu, vc_gpu = kcd.cpu().numpy(), vcd.cpu().numpy()
    for i, p in enumerate(positions):
        qq = q[i].reshape(hq, d).astype(np.float64)
        kk = k[i].reshape(hkv, d).astype(np.float64)
        if rope:
            c, s = decode_ref.rope_tables(d, np.array([p]), theta)   # the reference's float32 angles
            qq = decode_ref.apply_rope(qq, c[0].astype(np.float64), s[0].astype(np.float64))
            kk = decode_ref.apply_rope(kk, c[0].astype(np.float64), s[0].astype(np.float64))
        ulp = np.abs(np.spacing(kk.astype(np.float16))).astype(np.float64)
        assert np.all(np.abs(kc_gpu[i, :, p].astype(np.float64) - kk) <= ulp), "appended key"
        assert np.array_equal(vc_gpu[i, :, p], v[i].reshape(hkv, d).astype(np.float16)), "appended value"
        # untouched elsewhere
        mask = np.ones(max_pos, bool)
        mask[p] = False
        assert np.array_equal(kc_gpu[i][:, mask], kc[i][:, mask])
        ref = decode_ref.decode_attention_f64(qq, kc_gpu[i], vc_gpu[i], p + 1)
        tol = 1e-3 if out_dtype == torch.float32 else 1e-2
        check_close(got[i].reshape(hq, d), ref, f"attention b={i} pos={p}", tol=tol)
    return got


@pytest.mark.parametrize("positions", [[0], [5, 700], [255, 256], [511, 1023], [31, 32, 33, 95]])
def test_decode_attention_llama_heads(positions):
    print(f"decode attention positions {positions}", flush=True)
    _attention_case(len(positions), 32, 8, 128, 1024, positions, 500000.0, True, seed=sum(positions) + 1)


@pytest.mark.parametrize("hq,hkv,d,rope", [(8, 8, 64, True), (16, 2, 64, False), (16, 8, 128, True), (64, 8, 128, True)])
def test_decode_attention_shapes(hq, hkv, d, rope):
    print(f"decode attention hq={hq} hkv={hkv} d={d} rope={rope}", flush=True)
    _attention_case(3, hq, hkv, d, 600, [0, 299, 599], 10000.0, rope, seed=hq + d)


def test_decode_attention_long_cache_multi_step_waves():
    """A cache of 40000 positions: each wave walks two 32-position steps
    (online rescaling inside the wave) and 625 waves meet in the merge."""
    print("decode attention max_pos 40000", flush=True)
    _attention_case(2, 8, 2, 64, 40000, [39999, 12345], 500000.0, True, seed=40)


def test_decode_attention_batch16():
    """16 sequences (the batch-16 decode step's attention launch: 16 x 8 kv
    heads x 35 one-wave splits), positions at and around the 32-position split
    edges, one per sequence."""
    positions = [0, 31, 32, 63, 64, 95, 100, 255, 256, 511, 700, 1023, 1050, 1087, 1099, 5]
    print("decode attention batch 16 max_pos 1100", flush=True)
    _attention_case(16, 32, 8, 128, 1100, positions, 500000.0, True, seed=16)


def test_decode_attention_bf16_out_and_invalid_position():
    print("decode attention bf16 out", flush=True)
    _attention_case(2, 32, 8, 128, 512, [17, 300], 500000.0, True, seed=9, out_dtype=torch.bfloat16)
    # a position outside the cache: no cache write, NaN output
    kc = torch.zeros((1, 2, 64, 64), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    q = torch.ones((1, 4 * 64), device="cuda")
    k = torch.ones((1, 2 * 64), device="cuda")
    for bad in (64, -1):
        out = decode_attention(q, k, k.clone(), kc, vc, torch.tensor([bad], dtype=torch.int32, device="cuda"), 4, 2)
        assert torch.isnan(out).all()
        assert not kc.any() and not vc.any()


def test_decode_attention_sequence_of_steps_reuses_workspace():
    """Eight consecutive tokens through one workspace: every step's merge
    counters must have been reset by the previous one."""
    b, hq, hkv, d, max_pos = 2, 32, 8, 128, 2048
    rng = np.random.default_rng(4)
    kcd = torch.zeros((b, hkv, max_pos, d), dtype=torch.float16, device="cuda")
    vcd = torch.zeros_like(kcd)
    ws = DecodeAttentionWorkspace(b, hq, hkv, d, max_pos)
    tables = rope_tables(d, max_pos, 500000.0)
    start = np.array([0, 1000])
    for step in range(8):
        q = rng.standard_normal((b, hq * d)).astype(np.float32)
        k = rng.standard_normal((b, hkv * d)).astype(np.float32)
        v = rng.standard_normal((b, hkv * d)).astype(np.float32)
        pos = start + step
        print(f"decode attention step {step} positions {pos.tolist()}", flush=True)
        out = decode_attention(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                               kcd, vcd, torch.from_numpy(pos.astype(np.int32)).cuda(), hq, hkv, rope=tables,
                               workspace=ws).cpu().numpy()
        kc_gpu, vc_gpu = kcd.cpu().numpy(), vcd.cpu().numpy()
        for i in range(b):
            c, s = decode_ref.rope_tables(d, np.array([pos[i]]), 500000.0)
            qq = decode_ref.apply_rope(q[i].reshape(hq, d).astype(np.float64), c[0].astype(np.float64),
                                       s[0].astype(np.float64))
            ref = decode_ref.decode_attention_f64(qq, kc_gpu[i], vc_gpu[i], pos[i] + 1)
            check_close(out[i].reshape(hq, d), ref, f"step {step} b={i}")


@pytest.mark.parametrize("qtype,m", [(12, 1), (14, 1), (12, 3), (3, 1)])
def test_fused_rmsnorm_gemv_matches_norm_then_gemv(qtype, m):
    """The RMSNorm in the GEMV prologue (Q4_K / Q6_K, one token) or as its own
    launch (other cases): x_norm within one bf16 ulp of the standalone norm,
    outputs within the matmul bar of the fp64 product of that x_norm."""
    from dracort_amd.kernels import gguf_gemv_multi_rmsnorm, gguf_gemv_swiglu_rmsnorm
    from oracle import matmul_ref
    from tests.gguf_cases import quantized

    k = 4096 if qtype != 3 else 1024
    rng = np.random.default_rng(qtype + m)
    x = (rng.standard_normal((m, k)) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    ref_norm = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
    rms_norm(xd, wd, 1e-5, out_bf16=ref_norm)
    mats = [quantized(qtype, n, k, seed=n) for n in (512, 256)]
    outs = [torch.empty((m, n), device="cuda") for n in (512, 256)]
    xn = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
    print(f"fused rmsnorm multi type {qtype} m={m}", flush=True)
    gguf_gemv_multi_rmsnorm(xd, wd, 1e-5, xn, [(torch.from_numpy(b).cuda(), wt.shape[0]) for b, wt in mats], qtype, k,
                            outs)
    a, r = xn.float().cpu().numpy(), ref_norm.float().cpu().numpy()
    ulp = np.abs(np.spacing(r.astype(np.float32))) * 2 ** 16  # one bf16 ulp
    assert np.all(np.abs(a - r) <= ulp) and np.mean(a == r) > 0.99
    xs = xn.float().cpu().numpy()
    for (b, wt), y in zip(mats, outs):
        check_close(y.cpu().numpy(), matmul_ref.linear_ref(xs, wt), f"fused norm multi {qtype} m={m}")
    gb, gw = quantized(qtype, 1024, k, seed=5)
    ub, uw = quantized(qtype, 1024, k, seed=6)
    y = torch.empty((m, 1024), device="cuda")
    print(f"fused rmsnorm swiglu type {qtype} m={m}", flush=True)
    gguf_gemv_swiglu_rmsnorm(xd, wd, 1e-5, xn, torch.from_numpy(gb).cuda(), torch.from_numpy(ub).cuda(), qtype,
                             (1024, k), out=y)
    xs = xn.float().cpu().numpy()
    g = matmul_ref.linear_ref(xs, gw)
    check_close(y.cpu().numpy(), g / (1 + np.exp(-g)) * matmul_ref.linear_ref(xs, uw), f"fused norm swiglu {qtype}")
