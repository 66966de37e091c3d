"""Quantized weights on the device through the C ABI: syn_hip_matmul_q (the
activation quantizer, then the integer block dots) and syn_hip_embed over a
block-format table.

Pinned by the reference's kernel_golden.gguf (ggml's own quantized
activations of one x, bit for bit, and its vec_dot results for 8 rows of each
format, up to float re-association), then by the host restatement of the
formats (tests/quant_host.py, itself pinned by the same fixtures and by
quant_golden.gguf) on random blocks at model sizes: the activation bytes
must match bit for bit, each output within 1e-5 of sum |w| |x^| (the float
re-association bound), and the dequantized embedding rows bit for bit."""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np
import pytest

import quant_host as qh
from gpu_util import Arena, capi, check, lib
from synapse_amd.gguf import BLOCK, Q4_0, Q4_K, Q5_0, Q6_K, Q8_0, GGUFFile

pytestmark = pytest.mark.gpu
DATA = pathlib.Path(__file__).resolve().parent / "golden" / "reference"
KFORMATS = {"q4_0": Q4_0, "q5_0": Q5_0, "q8_0": Q8_0, "q4_K": Q4_K, "q6_K": Q6_K}
# Byte offsets of each format's binary16 scales inside a block.
SCALES = {Q4_0: (0,), Q5_0: (0,), Q8_0: (0,), Q4_K: (0, 2), Q6_K: (208,)}


@pytest.fixture(scope="module")
def arena():
    a = Arena(128 << 20)
    yield a
    a.close()


def random_blocks(t: int, rows: int, cols: int, rng) -> np.ndarray:
    """Random quants with finite binary16 scales of either sign."""
    bs, ts = BLOCK[t]
    raw = rng.integers(0, 256, size=(rows * (cols // bs), ts), dtype=np.uint8)
    for off in SCALES[t]:
        s = (rng.uniform(0.002, 0.05, raw.shape[0]) * rng.choice([-1, 1], raw.shape[0])).astype(np.float16)
        raw[:, off:off + 2] = s.view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


def matmul_q(arena: Arena, raw, t, x, rows, cols, bias=None):
    """Runs syn_hip_matmul_q; returns (out [n, rows], activation bytes)."""
    n = x.shape[0]
    mark = arena.top
    w_off = arena.put(raw)
    x_off = arena.put(np.ascontiguousarray(x, np.float32))
    act_bytes = int(lib().syn_hip_matmul_q_act_bytes(t, n, cols))
    act_off = arena.alloc(act_bytes)
    b_off = arena.put(bias) if bias is not None else capi.NO_OFFSET
    out_off = arena.alloc(n * rows * 4)
    d = capi.MatmulQDesc(w_offset=w_off, x_offset=x_off, act_offset=act_off, bias_offset=b_off, out_offset=out_off,
                         w_type=t, n=n, rows=rows, cols=cols)
    check(lib().syn_hip_matmul_q(arena.handle, ctypes.byref(d)))
    out = arena.download(out_off, (n, rows), np.float32)
    act = arena.download(act_off, (act_bytes,), np.uint8)
    arena.top = mark
    return out, act


@pytest.mark.parametrize("name", list(KFORMATS))
def test_matmul_q_matches_ggml_golden(arena, name):
    f = GGUFFile(DATA / "kernel_golden.gguf")
    t = KFORMATS[name]
    x = np.asarray(f.tensor("x"), np.float32).reshape(1, -1)
    raw, t_file, cols, rows = f.raw(f"{name}.w")
    want_act, _, _, _ = f.raw(f"{name}.act")
    y = np.asarray(f.tensor(f"{name}.y"), np.float32)
    assert t_file == t and x.shape[1] == cols
    out, act = matmul_q(arena, np.array(raw), t, x, rows, cols)
    assert np.array_equal(act, want_act), f"{name}: device activation bytes differ from ggml's"
    np.testing.assert_allclose(out[0], y, rtol=0, atol=1e-5 * max(1.0, float(np.abs(y).max())))


@pytest.mark.parametrize("t", [Q4_0, Q5_0, Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("n,rows,cols", [(1, 300, 2048), (3, 67, 4096), (2, 5, 256), (5, 9, 512), (1, 6, 20480),
                                         (31, 20, 512)])
def test_matmul_q_matches_host_blocks(arena, t, n, rows, cols):
    rng = np.random.default_rng(1000 * t + rows)
    raw = random_blocks(t, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    x[0, :7] = 0.0  # a run of zeros
    if n > 1:
        x[1, :256] = 0.0  # an all-zero block: d = 0, q = 0
    bias = rng.standard_normal(rows).astype(np.float32)
    out, act = matmul_q(arena, raw, t, x, rows, cols, bias)
    want_act = np.concatenate([qh.quantize_act(x[r], t) for r in range(n)])
    assert np.array_equal(act, want_act)
    w_all = qh.dequantize(raw, t).reshape(rows, cols).astype(np.float64)
    per_row = raw.size // rows
    act_rows = want_act.reshape(n, -1)
    for r in range(n):
        xa = qh.dequantize_act(act_rows[r], qh.act_type(t)).astype(np.float64)
        scale = np.abs(w_all) @ np.abs(xa)
        want = np.array([qh.vec_dot(raw[o * per_row:(o + 1) * per_row], t, act_rows[r]) for o in range(rows)])
        assert np.all(np.abs(out[r] - bias - want) <= 1e-5 * np.maximum(scale, 1.0)), (t, r)
        assert np.all(np.abs(out[r] - bias - w_all @ xa) <= 1e-5 * np.maximum(scale, 1.0)), (t, r)


@pytest.mark.parametrize("t", [Q4_0, Q5_0, Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("n,rows,cols", [(32, 37, 512), (70, 130, 2048), (64, 128, 4096), (33, 300, 256),
                                         (129, 33, 768), (40, 50, 800), (32, 1, 256), (65, 3, 512), (32, 2, 64)])
def test_matmul_q_gemm_matches_host(arena, t, n, rows, cols):
    """From 32 activation rows on, the product runs on the int8 matrix cores;
    the activation bytes stay ggml's bit for bit and every output is within
    1e-5 of sum |w| |x^| of the exact product of the dequantized operands
    (each block's integer sum is exact; only float association differs).
    800 columns (25 blocks, not whole two-block stages) take the 32-block
    formats' register kernel, the others their LDS kernels."""
    if cols % BLOCK[t][0]:
        pytest.skip("cols not whole blocks")
    rng = np.random.default_rng(7000 + 31 * t + n)
    raw = random_blocks(t, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    x[3, :256] = 0.0  # an all-zero block
    bias = rng.standard_normal(rows).astype(np.float32)
    out, act = matmul_q(arena, raw, t, x, rows, cols, bias)
    want_act = np.concatenate([qh.quantize_act(x[r], t) for r in range(n)])
    assert np.array_equal(act, want_act)
    w_all = qh.dequantize(raw, t).reshape(rows, cols).astype(np.float64)
    xa = np.stack([qh.dequantize_act(a, qh.act_type(t)) for a in want_act.reshape(n, -1)]).astype(np.float64)
    exact = xa @ w_all.T
    scale = np.abs(xa) @ np.abs(w_all).T
    err = np.abs(out.astype(np.float64) - bias - exact)
    assert np.all(err <= 1e-5 * np.maximum(scale, 1.0)), float((err / np.maximum(scale, 1.0)).max())


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 2048, 4096), (Q6_K, 1024, 14336), (Q8_0, 2048, 4096),
                                         (Q4_0, 2048, 4096), (Q5_0, 2048, 4096)])
def test_gemm_at_model_size_matches_the_gemv(arena, t, rows, cols):
    """Llama-3-8B row lengths (ffn_up's 4096 columns, ffn_down's 14336),
    128 activation rows: many workgroups in both dimensions and every stage
    of a long row (the row counts are cut to keep the host's bound quick). The GEMM (int8 matrix cores,
    LDS-staged) and the GEMV (v_dot4, one wave per row) are separate kernels
    over the same exact block integers, so they agree within twice the
    float-association bound, 2e-5 of sum |w| |x^|; the activation bytes are
    ggml's bit for bit."""
    rng = np.random.default_rng(9000 + t)
    raw = random_blocks(t, rows, cols, rng)
    n = 128
    x = rng.standard_normal((n, cols)).astype(np.float32)
    gemm, act = matmul_q(arena, raw, t, x, rows, cols)
    gemv = np.concatenate([matmul_q(arena, raw, t, x[i:i + 16], rows, cols)[0] for i in range(0, n, 16)])
    want_act = np.concatenate([qh.quantize_act(x[r], t) for r in range(n)])
    assert np.array_equal(act, want_act)
    w_abs = np.abs(qh.dequantize(raw, t).reshape(rows, cols))
    xa = np.abs(np.stack([qh.dequantize_act(a, qh.act_type(t)) for a in want_act.reshape(n, -1)]))
    scale = (xa @ w_abs.T).astype(np.float64)
    err = np.abs(gemm.astype(np.float64) - gemv.astype(np.float64))
    assert np.all(err <= 2e-5 * np.maximum(scale, 1.0)), float((err / np.maximum(scale, 1.0)).max())


@pytest.mark.parametrize("t", [Q4_0, Q5_0, Q8_0, Q4_K, Q6_K])
def test_embed_quantized_table_bit_exact(arena, t):
    rng = np.random.default_rng(7 + t)
    n_rows, size = 40, 512
    raw = random_blocks(t, n_rows, size, rng)
    tokens = np.array([0, 39, 5, 5, 17], np.uint32)
    mark = arena.top
    table = arena.put(raw)
    out = arena.alloc(len(tokens) * size * 4)
    d = capi.EmbedDesc(table_offset=table, out_offset=out, n_table_rows=n_rows, size=size, table_type=t)
    tk = (ctypes.c_uint32 * len(tokens))(*tokens.tolist())
    check(lib().syn_hip_embed(arena.handle, ctypes.byref(d), tk, len(tokens)))
    got = arena.download(out, (len(tokens), size), np.float32)
    arena.top = mark
    want = qh.dequantize(raw, t).reshape(n_rows, size)[tokens]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_matmul_q_rejects_bad_shapes(arena):
    d = capi.MatmulQDesc(w_offset=0, x_offset=0, act_offset=1 << 20, bias_offset=capi.NO_OFFSET,
                         out_offset=2 << 20, w_type=Q4_K, n=1, rows=4, cols=200)  # not whole super-blocks
    assert lib().syn_hip_matmul_q(arena.handle, ctypes.byref(d)) != 0
    d.cols, d.w_type = 256, 3  # an unknown format
    assert lib().syn_hip_matmul_q(arena.handle, ctypes.byref(d)) != 0
    d.w_type, d.act_offset = Q4_K, 0  # act overlaps w
    assert lib().syn_hip_matmul_q(arena.handle, ctypes.byref(d)) != 0
    assert lib().syn_hip_matmul_q_act_bytes(Q4_K, 2, 512) == 2 * 2 * 292
    assert lib().syn_hip_matmul_q_act_bytes(Q8_0, 1, 100) == 0
