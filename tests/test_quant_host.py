"""The host restatement of ggml's block formats against the reference's own
fixtures: quant_golden.gguf (blocks and their dequantized values, written by
gguf-py) and kernel_golden.gguf (ggml's quantized activations of one x and
its vec_dot results for 8 weight rows of each format)."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

import quant_host as qh
from synapse_amd.gguf import BF16, F16, Q4_0, Q4_K, Q5_0, Q6_K, Q8_0, GGUFFile

DATA = pathlib.Path(__file__).resolve().parent / "golden" / "reference"
FORMATS = {"f16": F16, "bf16": BF16, "q4_0": Q4_0, "q5_0": Q5_0, "q8_0": Q8_0, "q8_0.3d": Q8_0, "q4_k": Q4_K,
           "q6_k": Q6_K}
KFORMATS = {"q4_0": Q4_0, "q5_0": Q5_0, "q8_0": Q8_0, "q4_K": Q4_K, "q6_K": Q6_K}


@pytest.mark.parametrize("name", list(FORMATS))
def test_dequantize_matches_gguf_py_bit_for_bit(name):
    f = GGUFFile(DATA / "quant_golden.gguf")
    raw, t, row, n_rows = f.raw(f"{name}.q")
    assert t == FORMATS[name]
    want = np.asarray(f.tensor(f"{name}.expected"), np.float32).reshape(-1)
    got = qh.dequantize(raw, t)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", list(KFORMATS))
def test_activation_quantizers_match_ggml_bit_for_bit(name):
    f = GGUFFile(DATA / "kernel_golden.gguf")
    x = np.asarray(f.tensor("x"), np.float32)
    want, t_act, _, _ = f.raw(f"{name}.act")
    assert t_act == qh.act_type(KFORMATS[name])
    assert np.array_equal(qh.quantize_act(x, KFORMATS[name]), want)


@pytest.mark.parametrize("name", list(KFORMATS))
def test_vec_dot_matches_ggml(name):
    """Up to float re-association, as the reference's own test holds it; and
    within the exact bound sum |w| |x - x^| of the float product."""
    f = GGUFFile(DATA / "kernel_golden.gguf")
    x = np.asarray(f.tensor("x"), np.float32)
    raw, t, row, n_rows = f.raw(f"{name}.w")
    act, t_act, _, _ = f.raw(f"{name}.act")
    y = np.asarray(f.tensor(f"{name}.y"), np.float32)
    per_row = raw.size // n_rows
    w_all = qh.dequantize(raw, t).reshape(n_rows, row)
    xa = qh.dequantize_act(act, t_act)
    for r in range(n_rows):
        got = qh.vec_dot(raw[r * per_row:(r + 1) * per_row], t, act)
        assert abs(got - y[r]) <= 1e-5 * max(1.0, abs(y[r])), (r, got, y[r])
        exact = float(np.dot(w_all[r].astype(np.float64), xa.astype(np.float64)))
        assert abs(got - exact) <= 1e-5 * max(1.0, np.sum(np.abs(w_all[r]) * np.abs(xa))), (r, got, exact)
        bound = float(np.sum(np.abs(w_all[r].astype(np.float64)) * np.abs(x - xa)))
        assert abs(got - float(np.dot(w_all[r].astype(np.float64), x))) <= bound * 1.001 + 1e-5
