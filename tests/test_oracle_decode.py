"""Pins the oracle's decode glue (no GPU needed): RMSNorm, RoPE and decode
attention against closed forms and invariants.

* RMSNorm: the float32 restatement against the fp64 formula; unit weight
  makes every row's mean square 1; scaling the input does not change the
  output (up to eps).
* RoPE: the float32 tables against fp64; position 0 is the identity; each
  (i, i + D/2) pair is rotated by pos * inv_freq[i] (a complex product), so
  pair norms are kept and rotating by p1 then p2 equals rotating by p1 + p2.
* Attention: brute-force loops; one key gives its value; equal keys give the
  mean of the values; GQA maps query head h to kv head h // (Hq / Hkv).
"""

import numpy as np

from oracle import decode_ref


def test_rms_norm_matches_fp64_and_invariants():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((5, 4096)) * 3).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    got = decode_ref.rms_norm(x, w, 1e-5)
    ref = decode_ref.rms_norm_f64(x, w, 1e-5)
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-6)) < 1e-5
    unit = decode_ref.rms_norm_f64(x, np.ones(4096), 0.0)
    assert np.allclose(np.mean(unit ** 2, axis=-1), 1.0)
    assert np.allclose(decode_ref.rms_norm_f64(x * 7.0, w, 0.0), decode_ref.rms_norm_f64(x, w, 0.0))


def test_rope_tables_and_rotation():
    d, theta = 128, 500000.0
    pos = np.array([0, 1, 17, 1000, 8191])
    c32, s32 = decode_ref.rope_tables(d, pos, theta)
    c64, s64 = decode_ref.rope_tables_f64(d, pos, theta)
    # float32 angles pos * inv_freq lose ~pos * 2^-24 rad
    assert np.max(np.abs(c32 - c64)) < 1e-3 and np.max(np.abs(s32 - s64)) < 1e-3
    assert np.array_equal(c64[0], np.ones(d // 2)) and np.array_equal(s64[0], np.zeros(d // 2))
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, d))
    y = decode_ref.apply_rope(x, c64[3], s64[3])
    # complex form: (x1 + i x2) * exp(i angle)
    z = (x[:, : d // 2] + 1j * x[:, d // 2:]) * np.exp(1j * pos[3] / theta ** (np.arange(0, d, 2) / d))
    assert np.allclose(y[:, : d // 2], z.real) and np.allclose(y[:, d // 2:], z.imag)
    n = lambda a: a[:, : d // 2] ** 2 + a[:, d // 2:] ** 2  # noqa: E731
    assert np.allclose(n(y), n(x))
    c1, s1 = decode_ref.rope_tables_f64(d, np.array([5, 12, 17]), theta)
    two = decode_ref.apply_rope(decode_ref.apply_rope(x, c1[0], s1[0]), c1[1], s1[1])
    assert np.allclose(two, decode_ref.apply_rope(x, c1[2], s1[2]))


def test_decode_attention_brute_force_and_special_cases():
    rng = np.random.default_rng(2)
    hq, hkv, d, n = 8, 2, 16, 9
    q = rng.standard_normal((hq, d))
    kc = rng.standard_normal((hkv, 12, d)).astype(np.float16)
    vc = rng.standard_normal((hkv, 12, d)).astype(np.float16)
    out = decode_ref.decode_attention_f64(q, kc, vc, n)
    for h in range(hq):
        g = h // (hq // hkv)
        s = [sum(float(q[h, i]) * float(kc[g, j, i]) for i in range(d)) / np.sqrt(d) for j in range(n)]
        e = np.exp(np.array(s) - max(s))
        p = e / e.sum()
        ref = sum(p[j] * vc[g, j].astype(np.float64) for j in range(n))
        assert np.allclose(out[h], ref, rtol=1e-12, atol=1e-12)
    # one key: the output is that key's value
    one = decode_ref.decode_attention_f64(q, kc, vc, 1)
    assert np.allclose(one, np.repeat(vc[:, 0].astype(np.float64), hq // hkv, axis=0))
    # equal keys: the mean of the values
    ke = np.repeat(kc[:, :1], 12, axis=1)
    mean = decode_ref.decode_attention_f64(q, ke, vc, n)
    assert np.allclose(mean, np.repeat(vc[:, :n].astype(np.float64).mean(axis=1), hq // hkv, axis=0))


def test_decode_step_attention_appends_rotated_float16():
    rng = np.random.default_rng(3)
    hq, hkv, d, pos = 4, 2, 8, 5
    kc = np.zeros((hkv, 16, d), np.float16)
    vc = np.zeros((hkv, 16, d), np.float16)
    kc[:, :pos] = rng.standard_normal((hkv, pos, d))
    vc[:, :pos] = rng.standard_normal((hkv, pos, d))
    q = rng.standard_normal((hq, d)).astype(np.float32)
    k = rng.standard_normal((hkv, d)).astype(np.float32)
    v = rng.standard_normal((hkv, d)).astype(np.float32)
    out = decode_ref.decode_step_attention(q, k, v, kc, vc, pos, 10000.0)
    c, s = decode_ref.rope_tables_f64(d, np.array([pos]), 10000.0)
    assert np.array_equal(kc[:, pos], decode_ref.apply_rope(k.astype(np.float64), c[0], s[0]).astype(np.float16))
    assert np.array_equal(vc[:, pos], v.astype(np.float16))
    qr = decode_ref.apply_rope(q.astype(np.float64), c[0], s[0])
    assert np.allclose(out, decode_ref.decode_attention_f64(qr, kc, vc, pos + 1))
