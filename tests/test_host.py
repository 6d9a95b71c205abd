"""Host-side tests (no GPU): the C ABI library loads and exports every symbol
the header declares, argument errors map onto the reference's exception
classes without launching anything, and the host logic (quantizers, format
helpers, backend registry) behaves."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from dracort_amd import _native
from dracort_amd.exceptions import DracoFormatError
from dracort_amd.format import gguf as fmt
from dracort_amd.quantization import quantize
from oracle import gguf_ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "draco_gguf.h")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(draco_gguf_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    declared = _declared_symbols()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.SIGNATURES), "ctypes signatures must cover the header exactly"
    assert lib.draco_gguf_abi_version() == _native.ABI_VERSION


@pytest.mark.parametrize("qtype,expect", [
    (2, (32, 18)), (3, (32, 20)), (6, (32, 22)), (7, (32, 24)), (8, (32, 34)), (15, (256, 258)),
    (10, (256, 84)), (11, (256, 110)), (12, (256, 144)), (13, (256, 176)), (14, (256, 210)),
    (10 | 0x100, (256, 84)), (11 | 0x100, (256, 110)), (14 | 0x100, (256, 210))])
def test_block_info(qtype, expect):
    assert _native.block_info(qtype) == expect
    assert fmt.layout(qtype) == expect


def test_block_info_rejects_unknown_types():
    # F32 / F16 are not block types; 4, 5 were removed from ggml; 9 (Q8_1) and
    # 16+ (IQ*) are not read by the reference; the order flag only fits Q2_K / Q3_K / Q6_K
    for bad in (0, 1, 4, 5, 9, 16, 28, 8 | 0x100, 12 | 0x100, 13 | 0x100, 15 | 0x100):
        with pytest.raises(DracoFormatError):
            _native.block_info(bad)
        with pytest.raises(DracoFormatError):
            fmt.layout(bad)


FAKE = 0x10000  # aligned, never dereferenced: every call below fails validation first


def _dq(qtype, blocks, nbytes, out, n, k):
    return _native.load().draco_gguf_dequant_f32(qtype, blocks, nbytes, out, n, k, None)


def test_error_codes_before_launch():
    lib = _native.load()
    assert _dq(16, FAKE, 1 << 20, FAKE, 4, 256) == _native.DRACO_EINVAL_QTYPE
    assert "not supported" in _native.last_error()
    assert _dq(12, FAKE, 1 << 20, FAKE, 4, 300) == _native.DRACO_EINVAL_SHAPE          # K % 256
    assert _dq(12, FAKE, 4 * 144 - 1, FAKE, 4, 256) == _native.DRACO_EINVAL_SHAPE      # truncated payload
    assert "bytes" in _native.last_error()
    assert _dq(12, None, 1 << 20, FAKE, 4, 256) == _native.DRACO_EINVAL_ARG            # NULL
    assert _dq(12, FAKE + 4, 1 << 20, FAKE, 4, 256) == _native.DRACO_EINVAL_ARG        # misaligned
    assert _dq(12, FAKE, 1 << 20, FAKE, 0, 256) == _native.DRACO_EINVAL_SHAPE          # empty
    gemv = lib.draco_gguf_gemv
    assert gemv(12, FAKE, 1 << 20, FAKE, 1, None, FAKE, 17, 4, 256, None) == _native.DRACO_EINVAL_SHAPE  # M > 16
    assert gemv(12, FAKE, 1 << 20, FAKE, 1, None, FAKE, 0, 4, 256, None) == _native.DRACO_EINVAL_SHAPE
    assert gemv(12, FAKE, 1 << 20, FAKE, 7, None, FAKE, 1, 4, 256, None) == _native.DRACO_EINVAL_ARG    # dtype
    assert lib.draco_gguf_gemm(8, FAKE, 10, FAKE, None, FAKE, 64, 4, 64, None, 0, None) == _native.DRACO_EINVAL_SHAPE
    # prefill GEMM workspace: Q4_K needs f16 activations + three planes of 32-element sums + row scales
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    need = al(512 * 4096 * 2) + al(3 * 512 * 128 * 2) + al(512 * 4)
    # + room for split-K partial sums: S x N <= 128 x 256 / ceil(M / 256) (a few tiles split along K,
    # or a grid's partial last round split)
    assert lib.draco_gguf_gemm_workspace_size(12, 512, 4096) == need + 512 * 128 * 128 * 4
    assert lib.draco_gguf_gemm_workspace_size(12, 2048, 4096) == (al(2048 * 4096 * 2) + al(3 * 2048 * 128 * 2) +
                                                                  al(2048 * 4) + 2048 * 128 * 32 * 4)
    assert lib.draco_gguf_gemm_workspace_size(8, 512, 4096) == 0
    assert lib.draco_gguf_gemm_workspace_size(99, 512, 4096) == 0
    gemm = lib.draco_gguf_gemm
    assert gemm(12, FAKE, 1 << 30, FAKE, None, FAKE, 512, 64, 4096, FAKE, need - 1, None) == _native.DRACO_EWORKSPACE
    assert gemm(12, FAKE, 1 << 30, FAKE, None, FAKE, 512, 64, 4096, FAKE + 16, need, None) == _native.DRACO_EINVAL_ARG
    ptrs = (ctypes.c_void_p * 2)(FAKE, FAKE)
    moe = lib.draco_gguf_moe_ffn
    args = [12, ptrs, ptrs, ptrs, 1 << 30, FAKE, FAKE, 1, FAKE, 64, 256, 512, 2, 2, FAKE, 1 << 30, None]
    bad_k = list(args)
    bad_k[13] = 3  # top_k > n_experts
    assert moe(*bad_k) == _native.DRACO_EINVAL_SHAPE
    small_ws = list(args)
    small_ws[15] = 16
    assert moe(*small_ws) == _native.DRACO_EWORKSPACE
    trunc = list(args)
    trunc[4] = 100
    assert moe(*trunc) == _native.DRACO_EINVAL_SHAPE
    assert lib.draco_gguf_moe_workspace_size(64, 4096, 14336, 8, 2) > 64 * 2 * (4096 + 14336) * 4
    # fused decode launches
    w2 = (ctypes.c_void_p * 5)(*([FAKE] * 5))
    nb = (ctypes.c_size_t * 5)(*([1 << 20] * 5))
    nn = (ctypes.c_int64 * 5)(*([16] * 5))
    ys = (ctypes.c_void_p * 5)(*([FAKE + 0x100000] * 5))
    assert lib.draco_gguf_gemv_multi(12, 5, w2, nb, nn, ys, None, FAKE, 1, 1, 256, None) == _native.DRACO_EINVAL_ARG
    assert lib.draco_gguf_gemv_multi(12, 2, w2, nb, nn, None, None, FAKE, 1, 1, 256, None) == _native.DRACO_EINVAL_ARG
    assert lib.draco_gguf_gemv_swiglu(12, FAKE, FAKE, 1 << 20, FAKE, 1, None, None, 1, 16, 256, None) \
        == _native.DRACO_EINVAL_ARG
    # x overlapping the residual it updates
    assert lib.draco_gguf_gemv_residual(12, FAKE, 1 << 20, FAKE + 0x1000, 0, FAKE + 0x1000, None, 1, 16, 256,
                                        None) == _native.DRACO_EINVAL_ARG
    assert "overlap" in _native.last_error()


def test_check_maps_codes_to_reference_exceptions():
    _dq(16, FAKE, 1 << 20, FAKE, 4, 256)
    with pytest.raises(DracoFormatError):
        _native.check(_native.DRACO_EINVAL_QTYPE, "x")
    with pytest.raises(ValueError):
        _native.check(_native.DRACO_EINVAL_ARG, "x")
    from dracort_amd.exceptions import KernelError
    with pytest.raises(KernelError):
        _native.check(_native.DRACO_EHIP, "x")


def test_operators_refuse_cpu_tensors():
    from dracort_amd.kernels import gguf_dequantize, gguf_linear
    q = torch.zeros(144, dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU"):
        gguf_dequantize(q, 12, (1, 256))
    with pytest.raises(ValueError, match="GPU"):
        gguf_linear(torch.zeros(1, 256), q, 12, (1, 256))


def test_format_helpers():
    assert fmt.row_bytes(12, 4096) == 16 * 144
    assert fmt.tensor_bytes(14, (4096, 14336)) == 4096 * 56 * 210
    with pytest.raises(DracoFormatError):
        fmt.row_bytes(2, 48)
    assert fmt.BITS_PER_WEIGHT[12] == 4.5


# --- quantizers (product code, run on the CPU here) ---------------------------

def test_q8_0_q4_0_quantizers_reproduce_reference_encoder_bytes():
    from dracort_amd.quantization import quantize_q4_0, quantize_q8_0
    z = np.load(os.path.join(GOLDEN, "gguf_encoder_golden.npz"))
    for tag in ("small", "wide", "zero"):
        x = torch.from_numpy(z[f"x_{tag}"]).reshape(-1, 32)
        assert np.array_equal(quantize_q8_0(x).numpy(), z[f"q8_0_{tag}"])
        assert np.array_equal(quantize_q4_0(x).numpy(), z[f"q4_0_{tag}"])


@pytest.mark.parametrize("qtype,tol", [(12, 0.6), (14, 0.55)])
def test_k_quantizers_round_trip(qtype, tol):
    """Error per element within `tol` quantization steps of its sub-block."""
    from dracort_amd.quantization import quantize
    rng = np.random.default_rng(1)
    w = (rng.normal(size=(16, 1024)) * 0.02).astype(np.float32)
    w[3] *= 4.0
    blocks = quantize(torch.from_numpy(w), qtype).numpy()
    assert blocks.size == fmt.tensor_bytes(qtype, w.shape)
    dq = gguf_ref.dequantize_matrix(qtype, blocks, w.shape)
    sub = 32 if qtype == 12 else 16
    span = w.reshape(-1, sub)
    if qtype == 12:
        step = (span.max(1) - np.minimum(span.min(1), 0)) / 15
    else:
        step = np.abs(span).max(1) / 31
    err = np.abs(dq - w).reshape(-1, sub).max(1)
    # the 6-/8-bit rounding of the sub-block scales adds a few percent of a step
    assert np.all(err <= tol * step + 2e-4 * np.abs(w).max()), float((err / step).max())


def test_q6k_quantizer_d_last_layout():
    from dracort_amd.quantization import quantize
    w = torch.from_numpy((np.random.default_rng(2).normal(size=(4, 512)) * 0.02).astype(np.float32))
    ref = quantize(w, 14).numpy()
    up = quantize(w, 14 | 0x100).numpy()
    assert np.array_equal(gguf_ref.q6k_reorder(ref, to_upstream=True), up)


def test_registry_has_gguf_backend():
    from dracort_amd.quantization import QUANT_REGISTRY, GGUFBackend
    be = QUANT_REGISTRY.get("GGUF")
    assert isinstance(be, GGUFBackend) and "gguf" in QUANT_REGISTRY
    info = be.get_kernel_info()
    assert info["gpu_kernel"] and info["arch"] == "gfx950"
    assert be.supports_gpu_kernel(torch.device("cuda"))
    assert be.estimate_memory(4096 * 4096, 4) == 4096 * 4096 * 9 // 16


def test_gpu_tier_selection_rules():
    from dracort_amd.format.gguf import GgufTensorInfo
    from dracort_amd.runtime import GGUFGpuKernel, is_gguf_block_tensor

    k = GGUFGpuKernel()
    assert k.tier == "gpu-gguf" and k.name == "mi355x-gguf"
    assert k.supports(None) and not k.supports("int8_sym")
    assert is_gguf_block_tensor(GgufTensorInfo("w", 12, (16, 256)))
    assert is_gguf_block_tensor(GgufTensorInfo("w", 14 | 0x100, (16, 256)))
    assert not is_gguf_block_tensor(GgufTensorInfo("w", 0, (16, 256)))          # float32
    assert is_gguf_block_tensor(GgufTensorInfo("w", 3, (16, 256)))              # Q4_1
    assert is_gguf_block_tensor(GgufTensorInfo("w", 11 | 0x100, (16, 256)))     # Q3_K, ggml order
    assert not is_gguf_block_tensor(GgufTensorInfo("w", 9, (16, 256)))          # Q8_1: not read by the reference
    assert not is_gguf_block_tensor(GgufTensorInfo("w", 12, (4096,)))           # not 2-D
    assert not is_gguf_block_tensor(GgufTensorInfo("w", 12, (16, 256), quantization="int8_sym"))


def test_quantizers_match_reference_encoders_for_q4_1_q5_0_q5_1():
    """The package's Q4_1 / Q5_0 / Q5_1 bytes are the reference test encoders'
    (restated in oracle.encoders, tests/format/test_gguf.py:172-229)."""
    from oracle import encoders

    w = (np.random.default_rng(12).standard_normal((6, 256)) * 0.7).astype(np.float32)
    w[2] = 0.0          # zero span: d = 1
    w[3, :32] = 1.25    # constant block
    for qtype, enc in ((3, encoders.enc_q4_1), (6, encoders.enc_q5_0), (7, encoders.enc_q5_1)):
        got = quantize(torch.from_numpy(w), qtype).numpy()
        assert np.array_equal(got, np.frombuffer(enc(w.reshape(-1)), np.uint8)), qtype


@pytest.mark.parametrize("qtype", [10, 11, 14])
def test_quantizer_ggml_order_is_the_field_move(qtype):
    w = (np.random.default_rng(qtype).standard_normal((4, 512)) * 0.02).astype(np.float32)
    ref = quantize(torch.from_numpy(w), qtype).numpy()
    up = quantize(torch.from_numpy(w), qtype | 0x100).numpy()
    assert np.array_equal(gguf_ref.to_ggml_order(qtype, ref), up)


@pytest.mark.parametrize("qtype,tol", [(3, 0.08), (6, 0.06), (7, 0.04), (15, 0.01), (10, 0.45), (11, 0.25),
                                       (13, 0.05)])
def test_quantizers_round_trip(qtype, tol):
    """Quantize -> oracle dequantize stays within each format's resolution (rms, relative)."""
    w = (np.random.default_rng(qtype).standard_normal((16, 1024)) * 0.02).astype(np.float32)
    b = quantize(torch.from_numpy(w), qtype).numpy()
    deq = gguf_ref.dequantize_matrix(qtype, b, w.shape)
    rms = np.sqrt(np.mean((deq - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    assert rms < tol, (qtype, rms)


def test_decode_glue_validation_before_launch():
    """Shape and pointer checks of the glue entry points fail before any launch."""
    lib = _native.load()
    ws = lib.draco_gguf_decode_attention_workspace_size(1, 32, 8, 128, 1024)
    assert ws > 0
    assert lib.draco_gguf_decode_attention_workspace_size(1, 12, 8, 128, 1024) == 0  # not a multiple
    args = dict(q=FAKE, k=FAKE, v=FAKE, kc=FAKE, vc=FAKE, pos=FAKE)

    def call(hq, hkv, d, max_pos, ws_bytes=1 << 30, cos=None, sin=None):
        return lib.draco_gguf_decode_attention(args["q"], args["k"], args["v"], args["kc"], args["vc"], args["pos"],
                                               1, hq, hkv, d, max_pos, cos, sin, FAKE, 0, FAKE, ws_bytes, None)
    assert call(12, 8, 128, 64) == _native.DRACO_EINVAL_SHAPE     # query heads not a multiple of kv heads
    assert call(32, 8, 97, 64) == _native.DRACO_EINVAL_SHAPE      # odd head_dim
    assert call(32, 8, 258, 64) == _native.DRACO_EINVAL_SHAPE     # head_dim above 256
    # other head_dims and groups run the generic kernel, whose workspace holds the scores
    assert lib.draco_gguf_decode_attention_workspace_size(2, 12, 4, 96, 1000) == 2 * 12 * 1000 * 4
    assert lib.draco_gguf_decode_attention_workspace_size(1, 4, 2, 4, 64) == 4 * 64 * 4
    assert call(32, 8, 128, 1 << 25) == _native.DRACO_EINVAL_SHAPE
    assert call(32, 8, 128, 64, cos=FAKE) == _native.DRACO_EINVAL_ARG
    assert call(32, 8, 128, 64, ws_bytes=16) == _native.DRACO_EWORKSPACE
    assert lib.draco_gguf_rms_norm(FAKE, FAKE, 1e-5, FAKE, None, 1, 6, None) == _native.DRACO_EINVAL_SHAPE
    assert lib.draco_gguf_rms_norm(FAKE, FAKE, 1e-5, None, None, 1, 8, None) == _native.DRACO_EINVAL_ARG


def test_gpu_tier_cache_keys_separate_files_orders_and_bytes(tmp_path):
    """Two files with the same tensor names and offsets but different bytes,
    and one file read in both Q6_K field orders, never share a residency key;
    neither do two matmul() calls handed different weight bytes."""
    import time

    from dracort_amd.format.gguf_file import GGUFFile
    from dracort_amd.runtime.gpu_tier import bytes_weight_key, linear_weight_key
    from tests.gguf_writer import write_gguf

    rng = np.random.default_rng(3)
    payloads = [rng.integers(0, 256, 210 * 4, dtype=np.uint8).tobytes() for _ in range(2)]
    paths = []
    for i, p in enumerate(payloads):
        path = str(tmp_path / f"m{i}.gguf")
        write_gguf(path, [("general.architecture", "str", "llama")], [("blk.0.ffn_down.weight", (4, 256), 14, p)])
        paths.append(path)
    keys = set()
    for path in paths:
        for order in ("reference", "ggml"):
            with GGUFFile(path, field_order=order) as f:
                t = f.tensor("blk.0.ffn_down.weight")
                keys.add(linear_weight_key(f, t.info, t.kernel_type))
    assert len(keys) == 4
    # the same file reopened unchanged maps to the same key; rewritten, to a new one
    with GGUFFile(paths[0]) as f:
        t = f.tensor("blk.0.ffn_down.weight")
        k0 = linear_weight_key(f, t.info, t.kernel_type)
    with GGUFFile(paths[0]) as f:
        assert linear_weight_key(f, t.info, t.kernel_type) == k0
    time.sleep(0.01)
    write_gguf(paths[0], [("general.architecture", "str", "llama")],
               [("blk.0.ffn_down.weight", (4, 256), 14, payloads[1])])
    with GGUFFile(paths[0]) as f:
        assert linear_weight_key(f, f.tensor("blk.0.ffn_down.weight").info, 14) != k0
    info = t.info
    assert bytes_weight_key(info, 14, payloads[0]) != bytes_weight_key(info, 14, payloads[1])
    assert bytes_weight_key(info, 14, payloads[0]) == bytes_weight_key(info, 14, bytes(payloads[0]))
    assert bytes_weight_key(info, 14, payloads[0]) != bytes_weight_key(info, 14 | 0x100, payloads[0])
