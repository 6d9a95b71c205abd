"""GPU parity of the executor pieces and of whole GGUF models decoded on the GPU.

* dense float linear, embedding gather, SwiGLU, generic-shape decode
  attention and the row-spanning dequantization against the oracle;
* GPUExecutionBackend on GGUF files written with tests/gguf_writer.py -- a
  llama-shaped model (head_dim 64, Q4_K / Q6_K / Q8_0 projections, F16
  embeddings), a sparse-MoE model (3-D Q4_K expert stacks, F32 router) and the
  reference's own end-to-end fixture (qwen2, head_dim 4, Q8_0 [32, 16]
  weights whose blocks run across rows) -- against the fp64 oracle chain
  (oracle.model_ref, float16 KV rounding as the GPU cache stores it) at 1e-3,
  and against the unrounded chain / the fixture's unquantized weights at the
  reference's own bar allclose(atol=1e-2, rtol=1e-2) (tests/format/test_gguf.py:762);
* the fused, graph-captured DecodeStep built from the same llama GGUF file."""

import numpy as np
import pytest
import torch

from dracort_amd.kernels import dense_linear, get_rows, gguf_dequantize, swiglu
from oracle import gguf_ref, matmul_ref, model_ref
from tests.gguf_cases import Q4_K, Q6_K, Q8_0, check_close, quantized
from tests.gguf_models import write_llama, write_reference_tiny

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("wtype", [0, 1, 30])
@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_dense_linear(wtype, xdtype):
    rng = np.random.default_rng(wtype)
    for m, n, k in ((1, 37, 64), (5, 256, 130), (19, 64, 512)):  # k = 130: the element-wise path
        w32 = rng.standard_normal((n, k)).astype(np.float32)
        wt = {0: torch.float32, 1: torch.float16, 30: torch.bfloat16}[wtype]
        w = torch.from_numpy(w32).to(wt)
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(xdtype)
        b = torch.from_numpy(rng.standard_normal(n).astype(np.float32))
        ref = x.double().numpy() @ w.double().numpy().T + b.numpy()
        print(f"dense_linear type {wtype} x {xdtype} m={m} [{n},{k}]", flush=True)
        y = dense_linear(x.cuda(), w.cuda(), wtype, (n, k), bias=b.cuda())
        check_close(y.cpu().numpy(), ref, f"dense {wtype} [{n},{k}]", tol=1e-4)
        acc = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32))
        y2 = dense_linear(x.cuda(), w.cuda(), wtype, (n, k), out=acc.clone().cuda(), accumulate=True)
        check_close(y2.cpu().numpy(), acc.numpy() + ref - b.numpy(), f"dense accumulate {wtype}", tol=1e-4)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q8_0, Q6_K | 0x100, 3, 11])
def test_get_rows_block_tables_bit_exact(qtype):
    blocks, w = quantized(qtype, 96, 512, 7)
    ids = np.array([5, 0, 95, 5, 17], dtype=np.int32)
    got = get_rows(torch.from_numpy(blocks).cuda(), qtype, (96, 512), torch.from_numpy(ids).cuda())
    got = got.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), w[ids].view(np.uint32))


def test_get_rows_float_tables_and_bad_ids():
    rng = np.random.default_rng(3)
    t32 = rng.standard_normal((40, 24)).astype(np.float32)
    ids = torch.tensor([3, 39, 0, -1, 40], dtype=torch.int32, device="cuda")
    for gt, dt in ((0, torch.float32), (1, torch.float16), (30, torch.bfloat16)):
        tab = torch.from_numpy(t32).to(dt)
        got = get_rows(tab.cuda(), gt, (40, 24), ids).cpu().numpy()
        assert np.array_equal(got[:3], tab.float().numpy()[[3, 39, 0]])
        assert np.isnan(got[3:]).all()  # ids outside the table give NaN rows
    blocks, _ = quantized(Q4_K, 8, 256, 1)
    bad = get_rows(torch.from_numpy(blocks).cuda(), Q4_K, (8, 256), torch.tensor([8, -3], dtype=torch.int32,
                                                                                  device="cuda"))
    assert torch.isnan(bad).all()


def test_swiglu_kernel():
    rng = np.random.default_rng(4)
    g = rng.standard_normal(1000).astype(np.float32) * 4
    u = rng.standard_normal(1000).astype(np.float32)
    y, yb = torch.empty(1000, device="cuda"), torch.empty(1000, dtype=torch.bfloat16, device="cuda")
    swiglu(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), out=y, out_bf16=yb)
    ref = matmul_ref.silu64(g.astype(np.float64)) * u
    assert np.max(np.abs(y.cpu().numpy() - ref) / np.maximum(np.abs(ref), 1e-3)) < 1e-5
    assert torch.equal(yb, y.to(torch.bfloat16))


def test_row_spanning_dequant_bit_exact():
    """K = 16 Q8_0 (two rows per block, the reference fixture's [32, 16]) and
    K = 48 Q4_0 (blocks straddle rows): bit-exact against the flat oracle."""
    for qtype, n, k in ((8, 32, 16), (2, 8, 48)):
        w = np.random.default_rng(n).standard_normal(n * k).astype(np.float32)
        from dracort_amd.quantization import quantize
        blocks = quantize(torch.from_numpy(w.reshape(-1, 32)), qtype).numpy()
        ref = gguf_ref.dequantize(qtype, blocks, n * k).reshape(n, k)
        got = gguf_dequantize(torch.from_numpy(blocks).cuda(), qtype, (n, k)).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (qtype, n, k)


@pytest.mark.parametrize("hq,hkv,d", [(4, 2, 4), (12, 4, 96), (6, 6, 32), (16, 1, 256)])
def test_generic_decode_attention(hq, hkv, d):
    """Shapes outside the fast kernels (head_dim other than 64 / 128, groups
    other than 1, 2, 4, 8) against the decode oracle, as the fast kernels are
    checked: appended key within a float16 ulp of the rotated key, value
    exact, the rest of the cache untouched, attention within 1e-3 (float32
    out) / 1e-2 (bf16 out) -- two sequences, at position 0 and past 256."""
    from tests.test_gpu_glue import _attention_case

    print(f"generic attention hq={hq} hkv={hkv} d={d}", flush=True)
    _attention_case(2, hq, hkv, d, 300, [0, 257], 10000.0, True, hq * d)
    _attention_case(1, hq, hkv, d, 64, [33], 10000.0, False, hq + d, out_dtype=torch.bfloat16)


def _executor(path, **kw):
    from dracort_amd.runtime import GPUExecutionBackend
    return GPUExecutionBackend(path, **kw)


def _spec(cfg, tied=False, experts=0, top_k=2):
    return model_ref.ModelSpec(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, heads=cfg.num_attention_heads,
                               kv_heads=cfg.num_key_value_heads, eps=cfg.rms_norm_eps, theta=cfg.rope_theta,
                               tied=tied, experts=experts, top_k=top_k)


def _all_positions(ex, prompt):
    s = ex.new_sequence()
    got = ex.forward_step(s, np.array(prompt), start_position=0, return_all_positions=True)
    ex.end_sequence(s)
    return got


def test_executor_llama_gguf_matches_oracle_chain(tmp_path):
    path = str(tmp_path / "llama.gguf")
    ref_w = write_llama(path, seed=1)
    ex = _executor(path, max_positions=64)
    spec = _spec(ex.config)
    prompt = [5, 77, 200, 3, 311]
    print("executor llama prompt", flush=True)
    got = _all_positions(ex, prompt)
    ref16 = model_ref.llama_forward(ref_w, spec, prompt, kv_dtype=np.float16)
    for t in range(len(prompt)):
        e, nw = check_close(got[t], ref16[t], f"llama logits position {t}")
        print(f"llama position {t}: elementwise {e:.2e}, normwise {nw:.2e}", flush=True)
    ref32 = model_ref.llama_forward(ref_w, spec, prompt)
    assert np.allclose(got, ref32, atol=1e-2, rtol=1e-2)


def test_executor_batched_decode_and_greedy(tmp_path):
    path = str(tmp_path / "llama2.gguf")
    ref_w = write_llama(path, seed=2, types={"v": 12, "down": 12}, out_type=None, embed_type=12, hidden=256,
                        heads=4, kv_heads=1, inter=512, vocab=256)  # tied Q4_K embeddings, head_dim 64, group 4
    ex = _executor(path, max_num_seqs=3, max_positions=32)
    assert ex.config.tie_word_embeddings
    spec = _spec(ex.config, tied=True)
    prompts = [[1, 2, 3], [9, 8], [100, 50, 25]]
    seqs = [ex.new_sequence() for _ in prompts]
    last = [ex.forward_step(s, np.array(p), 0) for s, p in zip(seqs, prompts)]
    for p, lg in zip(prompts, last):
        check_close(lg, model_ref.llama_forward(ref_w, spec, p, kv_dtype=np.float16)[-1], "tied llama")
    nxt = [int(np.argmax(lg)) for lg in last]
    batch = ex.forward_batch_decode(seqs, nxt, [len(p) for p in prompts])
    for i, p in enumerate(prompts):
        ref = model_ref.llama_forward(ref_w, spec, p + [nxt[i]], kv_dtype=np.float16)[-1]
        check_close(batch[i], ref, f"batched decode seq {i}")
    with pytest.raises(Exception):
        ex.forward_batch_decode(seqs[:1], [1], [0])  # position must follow the cache
    for s in seqs:
        ex.end_sequence(s)
    out = ex.generate_greedy([4, 5], 4)
    assert len(out) == 6 and all(0 <= t < 256 for t in out)


def test_executor_moe_gguf_matches_oracle_chain(tmp_path):
    path = str(tmp_path / "moe.gguf")
    ref_w = write_llama(path, seed=3, experts=4, top_k=2, hidden=256, inter=512, vocab=300, layers=2)
    ex = _executor(path, max_positions=32)
    assert ex.config.num_experts == 4 and ex.config.num_experts_per_tok == 2
    spec = _spec(ex.config, experts=4, top_k=2)
    prompt = [7, 8, 250, 9]
    print("executor moe prompt", flush=True)
    got = _all_positions(ex, prompt)
    ref16 = model_ref.llama_forward(ref_w, spec, prompt, kv_dtype=np.float16)
    for t in range(len(prompt)):
        check_close(got[t], ref16[t], f"moe logits position {t}")
    assert np.allclose(got, model_ref.llama_forward(ref_w, spec, prompt), atol=1e-2, rtol=1e-2)


def test_executor_runs_the_reference_tiny_fixture(tmp_path):
    """The reference's end-to-end GGUF fixture, prompt [1, 2, 3, 4]: logits
    within the reference's own bar of its independent reference (unquantized
    weights), and within 1e-3 of the oracle chain on the dequantized weights."""
    path = str(tmp_path / "tiny.gguf")
    ref_w, orig = write_reference_tiny(path)
    ex = _executor(path)
    cfg = ex.config
    assert (cfg.head_dim, cfg.vocab_size, cfg.rms_norm_eps) == (4, 32, pytest.approx(1e-6))
    s = ex.new_sequence()
    logits = ex.forward_step(s, np.array([1, 2, 3, 4]), start_position=0)
    spec = _spec(cfg)
    check_close(logits, model_ref.llama_forward(ref_w, spec, [1, 2, 3, 4], kv_dtype=np.float16)[-1], "tiny")
    expected = model_ref.llama_forward(orig, spec, [1, 2, 3, 4])[-1]
    assert logits.shape == (32,)
    assert np.allclose(logits, expected, atol=1e-2, rtol=1e-2)


def test_fused_decode_step_from_gguf(tmp_path):
    """layer_set_from_gguf + DecodeStep (bf16 activations between launches,
    one HIP graph) on the llama file, fed tokens through the embedding gather:
    within the reference's bar of the oracle chain, token after token."""
    from dracort_amd.format.gguf_file import GGUFFile
    from dracort_amd.runtime import DecodeStep, layer_set_from_gguf

    path = str(tmp_path / "llama3.gguf")
    ref_w = write_llama(path, seed=4, out_type=14)
    with GGUFFile(path) as f:
        ls, attn = layer_set_from_gguf(f, max_positions=32)
        from dracort_amd.runtime import gguf_executor_config
        spec = _spec(gguf_executor_config(f))
    step = DecodeStep(ls, m=1, attention=attn, start_position=0)
    prompt = [11, 22, 33, 44]
    step.set_tokens([prompt[0]])
    step.capture()
    for t, tok in enumerate(prompt):
        step.set_tokens([tok])
        got = step.replay().cpu().numpy()[0]
        ref = model_ref.llama_forward(ref_w, spec, prompt[:t + 1])[-1]
        e, nw = matmul_ref.rel_err(got, ref)
        print(f"fused step token {t}: elementwise {e:.2e}, normwise {nw:.2e}", flush=True)
        assert np.allclose(got, ref, atol=1e-2, rtol=1e-2) and nw < 1e-2
