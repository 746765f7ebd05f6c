"""CPU checks of the product library: it loads, exports every symbol the C ABI
header declares, and its host-side quantizers produce the oracle's bits."""
import os
import re

import numpy as np
import pytest

import oracle as O
from dwim_amd import device as D

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "dwim_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dwim_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = D.lib()
    names = _declared()
    assert len(names) >= 40
    for n in names:
        assert hasattr(L, n), n
    # and the Python mirror binds each of them
    from dwim_amd import model as M
    bound = set(D.SIGNATURES) | set(M.MODEL_SIGNATURES)
    assert set(names) == bound, set(names) ^ bound


def test_opening_without_a_gpu_fails_cleanly():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    with pytest.raises(D.DwimError):
        D.Hip(0)


def test_f16_conversions_match_the_oracle_exhaustively():
    for bits in range(0, 65536, 7):
        if bits & 0x7C00 == 0x7C00:
            continue
        assert D.from_f16(bits) == O.from_f16(bits)
    rng = np.random.default_rng(1)
    x = (rng.normal(0, 1, 5000) * 10.0 ** rng.uniform(-9, 6, 5000)).astype(np.float32)
    for v in x:
        assert D.to_f16(float(v)) == O.to_f16(float(v))


def test_cache_quantizer_matches_the_oracle():
    rng = np.random.default_rng(2)
    for scale in (1e-9, 1e-6, 1e-3, 1.0, 1e3, 1e6):
        for _ in range(50):
            b = (rng.normal(0, 1, 32) * scale).astype(np.float32)
            assert D.quantize_block(b)[0] == O.quantize(b)[0]
            assert np.array_equal(D.quantize_block(b)[1], O.quantize(b)[1])
    # the reference's edge blocks (gpu/tests.rs:705-714)
    for e in ([127.0, 0.5, 1.5, -2.5, 126.5, -0.0, 3.5000002, -3.4999998], [1e6, -1e6, 65504.0, 65520.0, 0.1],
              [1e-3, -3e-7, 2e-4, 1e-9], [1e-6, 7e-7, -3e-7], [1e-9, -1e-12], [0.0]):
        b = np.zeros(32, np.float32)
        b[:len(e)] = e
        s, q = D.quantize_block(b)
        so, qo = O.quantize(b)
        assert s == so and np.array_equal(q, qo)


@pytest.mark.parametrize("fmt", [D.Q4_0, D.Q8_0, D.Q4_K, D.Q6_K])
def test_weight_quantizers_match_the_oracle(fmt):
    rows, cols = 7, 1024
    vals = (O.Rng(9 + fmt).floats(rows * cols) * 0.05).reshape(rows, cols)
    vals[1] = 0.0
    vals[2, :300] = np.abs(vals[2, :300])
    t = D.Tensor.quantize(fmt, vals)
    w = O.Weight.quantized({D.Q4_0: O.Q4_0, D.Q8_0: O.Q8_0, D.Q4_K: O.Q4_K, D.Q6_K: O.Q6_K}[fmt], vals)
    assert np.array_equal(t.quants.view(np.uint8), w.quants.view(np.uint8))
    if w.scales is not None:
        assert np.array_equal(t.scales, w.scales)


def test_quantizers_match_the_golden_fixture():
    g = np.load(os.path.join(ROOT, "tests", "golden", "q4_k_q6_k.npz"))
    x = g["x"].reshape(1, -1)
    assert np.array_equal(D.Tensor.quantize(D.Q4_K, x).quants, g["q4_k"])
    assert np.array_equal(D.Tensor.quantize(D.Q6_K, x).quants, g["q6_k"])


def test_synthetic_values_are_deterministic_and_normal():
    a = D.synthetic_values(5, 0, 200000, 0.02)
    b = D.synthetic_values(5, 1000, 1000, 0.02)
    assert np.array_equal(a[1000:2000], b)
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    assert not np.array_equal(a[:1000], D.synthetic_values(6, 0, 1000, 0.02))


def test_synthetic_streams_match_the_oracles_restatement():
    for seed, first, sigma in ((1, 0, 0.02), (2 ** 63 + 5, 10 ** 9, 1.0), (77, 12345, 0.3)):
        assert np.array_equal(D.synthetic_values(seed, first, 4096, sigma),
                              O.synthetic_values(seed, first, 4096, sigma))


def test_selecting_rows_and_column_groups_reorders_every_format():
    # gpu/cpu.rs:455-509, dequantized through the oracle
    rows, cols = 3, 512
    w = O.Rng(5).floats(rows * cols).reshape(rows, cols)
    for fmt, ofmt in ((D.BF16, O.BF16), (D.Q4_0, O.Q4_0), (D.Q8_0, O.Q8_0), (D.Q4_K, O.Q4_K), (D.Q6_K, O.Q6_K)):
        t = D.Tensor.quantize(fmt, w)

        def deq(tt):
            return O.Weight(ofmt, tt.rows, tt.cols, tt.quants, tt.scales).dequantize()

        whole = deq(t)
        picked = t.select_rows([2, 0, 2])
        assert picked.shape == (3, cols)
        got = deq(picked)
        for i, r in enumerate([2, 0, 2]):
            assert np.array_equal(got[i], whole[r])
        swapped = t.select_column_groups(256, [1, 0])
        got = deq(swapped)
        assert np.array_equal(got[:, :256], whole[:, 256:])
        assert np.array_equal(got[:, 256:], whole[:, :256])
