"""Pins the oracle's KV-cache attention (oracle.cpp: kv_append, attend_group,
attention, the session's op_attention driver), restating
S/kernels/attention.hpp:147-269 and S/graph/session.hpp:348-374.

What pins it, without running the reference:
  * the reference's known answers: KV rows are the RNE binary16 of the input
    bit for bit, and at position 0 the output is exactly fp16(V)
    (tests/sdk/kernels_attention.cpp:178-240);
  * a double-precision brute force on f16-rounded q, K, V within 2e-3 (the
    reference's own bound), for every shape family -- it fixes the scale, the
    GQA head mapping h -> h / group and the causal horizon;
  * structure: head h reads only KV head h / group; token i of a run sees
    rows 0..pos+i only; a batched run equals token-by-token decoding bit for
    bit (tests/sdk/llama_prefill.cpp:20-52); results do not depend on the
    thread count (tests/sdk/llama_threads.cpp:32-58).
A planted mistake (a head read from the wrong KV group, a dropped f16
rounding of q, a causal off-by-one) fails at least one of these.
"""
from __future__ import annotations

import numpy as np
import pytest

import binding as orc


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _r16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def _brute(q, k_rows, v_rows, pos0, n_heads, n_kv, hd, scale):
    """Double precision on binary16-rounded operands: token i attends rows
    0..pos0+i, head h reads KV head h // (n_heads // n_kv)."""
    group = n_heads // n_kv
    out = np.zeros(q.shape, np.float64)
    K = _r16(k_rows).reshape(-1, n_kv, hd)
    V = _r16(v_rows).reshape(-1, n_kv, hd)
    for i in range(q.shape[0]):
        n_pos = pos0 + i + 1
        for h in range(n_heads):
            g = h // group
            s = K[:n_pos, g] @ _r16(q[i, h * hd:(h + 1) * hd]) * scale
            p = np.exp(s - s.max())
            out[i, h * hd:(h + 1) * hd] = (p / p.sum()) @ V[:n_pos, g]
    return out


def test_scratch_sizes_follow_the_reference():
    # attention_group_floats = group * (max_ctx + hd); scratch = n_kv slots
    assert orc.scratch_floats(32, 8, 128, 4097) == 8 * 4 * (4097 + 128)
    assert orc.lib().orc_attention_group_floats(4, 2, 16, 12) == 2 * (12 + 16)


def test_gqa_growing_cache_reference_case():
    """tests/sdk/kernels_attention.cpp:178-240 restated: n_heads 4, n_kv 2,
    hd 16, max_ctx 12, one decode step per position on one cache."""
    n_heads, n_kv, hd, max_ctx = 4, 2, 16, 12
    row = n_kv * hd
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    g = _rng(9)
    kc, vc = orc.new_cache(max_ctx, n_kv, hd)
    ks, vs = [], []
    for pos in range(max_ctx):
        q = g.standard_normal((1, n_heads * hd)).astype(np.float32)
        k = g.standard_normal((1, row)).astype(np.float32)
        v = g.standard_normal((1, row)).astype(np.float32)
        ks.append(k[0])
        vs.append(v[0])
        out = orc.attention_rows(q, k, v, pos, kc, vc, n_heads, scale)
        assert np.array_equal(kc[pos], k[0].astype(np.float16).view(np.uint16))
        assert np.array_equal(vc[pos], v[0].astype(np.float16).view(np.uint16))
        want = _brute(q, np.array(ks), np.array(vs), pos, n_heads, n_kv, hd, scale)
        assert np.max(np.abs(out - want)) < 2e-3
        if pos == 0:
            want0 = np.concatenate([vc[0].view(np.float16)[(h // 2) * hd:(h // 2 + 1) * hd] for h in range(n_heads)])
            assert np.array_equal(out[0], want0.astype(np.float32))


@pytest.mark.parametrize("n_heads,n_kv,hd,pos,n", [
    (8, 8, 32, 0, 32), (8, 8, 32, 32, 1), (32, 8, 128, 40, 1), (32, 8, 128, 0, 24), (12, 4, 96, 5, 9),
    (6, 3, 40, 0, 17), (4, 2, 12, 3, 6), (16, 1, 64, 0, 20), (8, 4, 256, 7, 3),
])
def test_attention_rows_match_double_brute_force(n_heads, n_kv, hd, pos, n):
    g = _rng(n_heads * 1000 + hd + pos)
    row = n_kv * hd
    total = pos + n
    q_all = g.standard_normal((total, n_heads * hd)).astype(np.float32)
    k_all = g.standard_normal((total, row)).astype(np.float32)
    v_all = g.standard_normal((total, row)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    kc, vc = orc.new_cache(total + 2, n_kv, hd)
    if pos:
        orc.attention_rows(q_all[:pos], k_all[:pos], v_all[:pos], 0, kc, vc, n_heads, scale)
    out = orc.attention_rows(q_all[pos:], k_all[pos:], v_all[pos:], pos, kc, vc, n_heads, scale)
    want = _brute(q_all[pos:], k_all, v_all, pos, n_heads, n_kv, hd, scale)
    assert np.max(np.abs(out - want)) < 2e-3


def test_each_query_head_reads_its_own_kv_group():
    """V constant per KV head and one cached position: head h's output is
    exactly fp16 of KV head h // group's constant."""
    n_heads, n_kv, hd = 12, 3, 16
    consts = np.array([0.75, -1.5, 2.25], np.float32)
    k = np.zeros((1, n_kv * hd), np.float32)
    v = np.repeat(consts, hd)[None, :]
    q = _rng(1).standard_normal((1, n_heads * hd)).astype(np.float32)
    kc, vc = orc.new_cache(4, n_kv, hd)
    out = orc.attention_rows(q, k, v, 0, kc, vc, n_heads, 0.25)
    for h in range(n_heads):
        assert np.all(out[0, h * hd:(h + 1) * hd] == consts[h // (n_heads // n_kv)])


def test_q_is_rounded_to_binary16_before_the_dot():
    """attend_group rounds q to f16 (S/kernels/attention.hpp:204-206): q and
    fp16(q) give identical outputs, bit for bit."""
    n_heads, n_kv, hd, n = 8, 2, 32, 10
    g = _rng(2)
    q = (g.standard_normal((n, n_heads * hd)) * 3).astype(np.float32)
    k = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    v = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    outs = []
    for qq in (q, q.astype(np.float16).astype(np.float32)):
        kc, vc = orc.new_cache(n, n_kv, hd)
        outs.append(orc.attention_rows(qq, k, v, 0, kc, vc, n_heads, 0.2))
    assert np.array_equal(outs[0], outs[1])


def test_normalised_probabilities_are_rounded_to_binary16():
    """attend_group rounds each normalised p to binary16 before p.V
    (S/kernels/attention.hpp:222-227). With one-hot V rows (V_t = e_t, t <
    hd) output element d is p_d times exactly 1, so every output element is
    a binary16 value, and element d equals the binary16 rounding of the
    double-precision softmax weight of position d to within one binary16
    step. Dropping that rounding leaves float weights, which are almost never
    binary16 values: the first assertion then fails."""
    n_heads, n_kv, hd, pos = 4, 2, 64, 39  # 40 positions attended
    g = _rng(7)
    n = pos + 1
    q = (g.standard_normal((n, n_heads * hd)) * 2).astype(np.float32)
    k = (g.standard_normal((n, n_kv * hd)) * 2).astype(np.float32)
    v = np.zeros((n, n_kv * hd), np.float32)
    for t in range(n):
        for kv in range(n_kv):
            v[t, kv * hd + t] = 1.0
    kc, vc = orc.new_cache(n, n_kv, hd)
    scale = 0.125
    out = orc.attention_rows(q, k, v, 0, kc, vc, n_heads, scale)[pos]  # the last token sees all 40 rows
    assert np.array_equal(out.astype(np.float16).astype(np.float32), out)
    group = n_heads // n_kv
    for h in range(n_heads):
        kv = h // group
        qh = q[pos, h * hd:(h + 1) * hd].astype(np.float16).astype(np.float64)
        kh = k[:, kv * hd:(kv + 1) * hd].astype(np.float16).astype(np.float64)
        s_ = kh @ qh * scale
        p_ = np.exp(s_ - s_.max())
        p_ /= p_.sum()
        got = out[h * hd:h * hd + n].astype(np.float64)
        step = np.abs(np.spacing(p_.astype(np.float16)).astype(np.float64))
        assert np.all(np.abs(got - p_) <= step), h
        assert np.all(out[h * hd + n:(h + 1) * hd] == 0.0)


def test_causal_horizon():
    """Changing rows after position p leaves tokens up to p unchanged, and
    changes token p + 1."""
    n_heads, n_kv, hd, n = 4, 2, 16, 12
    g = _rng(3)
    q = g.standard_normal((n, n_heads * hd)).astype(np.float32)
    k = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    v = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    outs = []
    for bump in (0.0, 1.0):
        kk, vv = k.copy(), v.copy()
        kk[7:] += bump
        vv[7:] -= bump
        kc, vc = orc.new_cache(n, n_kv, hd)
        outs.append(orc.attention_rows(q, kk, vv, 0, kc, vc, n_heads, 0.25))
    assert np.array_equal(outs[0][:7], outs[1][:7])
    assert not np.array_equal(outs[0][7], outs[1][7])


def test_batched_prefill_equals_token_by_token_bit_exact():
    n_heads, n_kv, hd, n = 8, 4, 32, 20
    g = _rng(4)
    q = g.standard_normal((n, n_heads * hd)).astype(np.float32)
    k = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    v = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    kc, vc = orc.new_cache(n, n_kv, hd)
    batched = orc.attention_rows(q, k, v, 0, kc, vc, n_heads, 0.125)
    kc2, vc2 = orc.new_cache(n, n_kv, hd)
    single = np.concatenate([orc.attention_rows(q[i:i + 1], k[i:i + 1], v[i:i + 1], i, kc2, vc2, n_heads, 0.125)
                             for i in range(n)])
    assert np.array_equal(batched, single)
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


@pytest.mark.parametrize("threads", [2, 3, 8])
def test_thread_count_does_not_change_results(threads):
    n_heads, n_kv, hd, n = 16, 8, 64, 9
    g = _rng(5)
    q = g.standard_normal((n, n_heads * hd)).astype(np.float32)
    k = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    v = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    outs = []
    for t in (1, threads):
        kc, vc = orc.new_cache(n, n_kv, hd)
        outs.append(orc.attention_rows(q, k, v, 0, kc, vc, n_heads, 0.125, threads=t))
    assert np.array_equal(outs[0], outs[1])


def test_attend_rows_is_the_attend_half():
    n_heads, n_kv, hd, n = 8, 2, 32, 6
    g = _rng(6)
    q = g.standard_normal((n, n_heads * hd)).astype(np.float32)
    k = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    v = g.standard_normal((n, n_kv * hd)).astype(np.float32)
    kc, vc = orc.new_cache(n, n_kv, hd)
    full = orc.attention_rows(q, k, v, 0, kc, vc, n_heads, 0.2)
    assert np.array_equal(orc.attend_rows(q, 0, kc, vc, n_heads, 0.2), full)
