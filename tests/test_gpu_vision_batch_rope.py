"""GPU parity: bidirectional (ViT) self-attention, ragged batched decode,
RoPE, and the C ABI's descriptor checks."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import binding as orc
from gpu_util import SYN_F16, SYN_F32, Arena, SeqDesc, capi, check, lib, put_rows, self_attention, seq_array
from helpers import assert_close, assert_p_rounded_normalised
from synapse_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def arena():
    a = Arena(3 << 30)
    yield a
    a.close()


# ---- bidirectional ----------------------------------------------------------

# f32 rows take a kernel with the reference's f32 arithmetic: the score and
# output fma chains in the oracle's order; the exponential (device expf) and
# the order of the double sum of the exponentials (per lane, then across
# lanes) differ, which moves only the last bits.
F32_BOUND = 2e-6


def _vision(arena, n, batch, n_heads, hd, dtype, sigma=0.5, seed=3, images=None):
    g = wl.rng(seed)
    shape = (batch * n, n_heads * hd)
    q, k, v = (wl.normal(g, shape, sigma) for _ in range(3))
    if dtype == SYN_F16:
        q, k, v = (x.astype(np.float16).astype(np.float32) for x in (q, k, v))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    got = self_attention(arena, q, k, v, n, batch, n_heads, scale, dtype)
    for b in (range(batch) if images is None else images):
        sl = slice(b * n, (b + 1) * n)
        want = orc.self_attention(q[sl], k[sl], v[sl], n_heads, scale, threads=8)
        assert_close(got[sl], want, what=f"image {b} n={n} heads={n_heads} hd={hd}")
        if dtype == SYN_F32:
            err = np.abs(got[sl] - want).max() / np.abs(want).max()
            assert err < F32_BOUND, (b, n, hd, err)


def test_vision_clip_vit_l14(arena):
    """Config 5 at full size: 32 images x 257 rows, 16 heads of 64, f16
    inputs ~ N(0, 0.5^2); every image checked against the oracle."""
    c = wl.C5
    _vision(arena, c.n, c.batch, c.n_heads, c.head_dim, SYN_F16, c.sigma, seed=wl.SEED)


@pytest.mark.parametrize("n,batch,n_heads,hd", [(257, 32, 16, 64), (257, 3, 5, 128), (1000, 2, 3, 64)])
def test_vision_is_deterministic(arena, n, batch, n_heads, hd):
    """Two launches on the same f16 inputs give the same bits. Config 5's
    shape (257 rows: the head-resident kernel with its tail rows summed in
    quarters across the waves), a head-resident shape at hd 128 and a tiled
    one. The reference pins split invariance bit for bit
    (tests/sdk/kernels_vision.cpp:252-263; tests/sdk/clip_golden.cpp:37-44)."""
    g = wl.rng(n + hd)
    shape = (batch * n, n_heads * hd)
    q, k, v = (wl.normal(g, shape, 0.5).astype(np.float16).astype(np.float32) for _ in range(3))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    a = self_attention(arena, q, k, v, n, batch, n_heads, scale, SYN_F16)
    b = self_attention(arena, q, k, v, n, batch, n_heads, scale, SYN_F16)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("n,hd", [(37, 8), (1, 8), (6, 16), (50, 24), (130, 64), (257, 128), (64, 256),
                                  (288, 64), (289, 64), (577, 64), (128, 128), (129, 128), (31, 96)])
def test_vision_shapes_f32_inputs(arena, n, hd):
    """The reference's self-attention cases (tests/sdk/kernels_vision.cpp:
    200-250, n in {37, 1, 6, 13, 50}) and larger images with f32 inputs,
    which keep the reference's f32 arithmetic: within F32_BOUND of the
    oracle."""
    _vision(arena, n, 2, 3, hd, SYN_F32)


def test_vision_f32_beyond_lds_rows(arena):
    """f32 images longer than the f32 kernel's 16384 rows take the
    matrix-core kernel, which rounds the operands to binary16 on load: four
    query rows against a float64 softmax, within binary16's rounding."""
    n, hd = 16400, 64
    g = wl.rng(21)
    q, k, v = (wl.normal(g, (n, hd), 0.5) for _ in range(3))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    got = self_attention(arena, q, k, v, n, 1, 1, scale, SYN_F32)
    for i in (0, 1, 8191, n - 1):
        s = (q[i].astype(np.float64) @ k.astype(np.float64).T) * scale
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ v.astype(np.float64)
        assert np.abs(got[i] - want).max() < 2e-3 * np.abs(want).max() + 1e-4, i


@pytest.mark.parametrize("n,hd", [(257, 64), (577, 64), (100, 128), (1, 64), (33, 32), (64, 64), (65, 64),
                                  (96, 96), (190, 96), (128, 128), (288, 64), (540, 32), (258, 64), (2, 64),
                                  (513, 32), (514, 32), (129, 96)])
def test_vision_many_heads_f16(arena, n, hd):
    """Several images and heads at once with f16 inputs: every (image, head)
    block of the grid is checked. With keys resident, f16 rows are staged in
    two halves (the first query tile runs over the first while the second
    lands): the shapes cover no second half (n <= 64), a second half ending
    in a lone 32-key slice (65, 96, 257) and the largest resident n per head
    size. A last query tile of one or two rows that would be a fifth tile of
    32 (257, 258, 1, 2, 513, 514, 129 rows) is computed on the vector units."""
    _vision(arena, n, 3, 5, hd, SYN_F16, seed=11)


def _tail_rows(arena, n, hd, batch, n_heads, images):
    g = wl.rng(n + hd)
    shape = (batch * n, n_heads * hd)
    q, k, v = (wl.normal(g, shape, 0.5).astype(np.float16).astype(np.float32) for _ in range(3))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    got = self_attention(arena, q, k, v, n, batch, n_heads, scale, SYN_F16)
    tiles = (n + 31) // 32
    first = 32 * (tiles - 1)
    has_tail = tiles % 4 == 1 and n - first <= 2  # 4 waves per block
    for b in images:
        sl = slice(b * n, (b + 1) * n)
        want = orc.self_attention(q[sl], k[sl], v[sl], n_heads, scale, threads=8)
        assert_close(got[sl], want, what=f"image {b} n={n} heads={n_heads} hd={hd}")
        if has_tail:
            tail = np.abs(got[sl][first:] - want[first:]).max() / np.abs(want).max()
            assert tail < 1e-5, (b, n, hd, tail)


@pytest.mark.parametrize("n,hd", [(257, 64), (258, 64), (1, 64), (2, 64), (513, 32), (514, 32), (1, 32),
                                  (129, 96), (2, 96), (1, 128), (2, 128)])
def test_vision_tail_rows_keep_f32_probabilities(arena, n, hd):
    """The vector-unit rows (the last tile's one or two rows) keep p in f32
    and sum in f32 over binary16-exact inputs, as the oracle does: within
    1e-5 of the largest output, where the matrix-core rows (p rounded to
    binary16) are held to the parity bound only. The block's four waves
    share them (keys scored across the block, output dims in 16-dim slices
    per wave, key quarters per 16-lane row), so a wrong key, a dropped key
    quarter, a wrong dim slice or a wrong head would miss by orders of
    magnitude; head dims 32 to 128 cover one and two 64-dim passes, with
    idle slices at 32 and 96. Few units: one per 4-wave block, tail rows
    when the query tiles are 1 mod 4."""
    _tail_rows(arena, n, hd, 2, 3, range(2))


@pytest.mark.parametrize("n,hd", [(257, 64), (258, 64), (100, 64), (2, 64), (513, 32), (64, 32), (289, 32)])
def test_vision_config5_grid(arena, n, hd):
    """32 images x 16 heads: config 5's grid of 512 blocks, two per CU, at
    other row counts (tail rows where the query tiles are 1 mod 4: 257, 258,
    2, 513). Images 0, 15 and 31 are checked whole."""
    _tail_rows(arena, n, hd, 32, 16, (0, 15, 31))


@pytest.mark.parametrize("n,hd", [(13, 12), (50, 20), (6, 4)])
def test_vision_generic_head_dims(arena, n, hd):
    _vision(arena, n, 1, 3, hd, SYN_F32)


# ---- ragged batched decode ---------------------------------------------------

def _ragged(arena, lengths, n_heads, n_kv, hd, seed, repeats=1):
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    g = wl.rng(seed)
    row = n_kv * hd
    mark = arena.top
    seqs, refs = [], []
    for L in lengths:
        kc = wl.to_f16_bits(wl.rope_rows(wl.normal(g, (L, row)), hd, 0, 500000.0))
        vc = wl.to_f16_bits(wl.normal(g, (L, row)))
        q = wl.normal(g, (1, n_heads * hd))
        cache = capi.kv_state(arena, L, n_kv, hd)
        capi.upload_cache(arena, cache, kc, vc)
        q_off = put_rows(arena, q, SYN_F32)
        out_off = arena.alloc(n_heads * hd * 4)
        seqs.append(SeqDesc(cache=cache, q_offset=q_off, out_offset=out_off, pos=L - 1))
        ok_k, ok_v = kc, vc
        refs.append(orc.attend_rows(q, L - 1, ok_k, ok_v, n_heads, scale, threads=8))
    arr = seq_array(seqs)
    need = int(lib().syn_hip_attend_batch_scratch_bytes(arr, len(seqs), n_heads))
    scratch = arena.alloc(max(need, 256))
    runs = []
    for _ in range(repeats):
        check(lib().syn_hip_attend_batch(arena.handle, arr, len(seqs), n_heads, scale, SYN_F32, scratch, need))
        runs.append([arena.download(s.out_offset, (1, n_heads * hd), np.float32) for s in seqs])
    for i, got in enumerate(runs[0]):
        assert_close(got, refs[i], what=f"sequence {i} (length {lengths[i]})")
        if lengths[i] <= SHORT_ROWS:
            assert_p_rounded_normalised(got, refs[i], n_heads, what=f"sequence {i} (length {lengths[i]})")
    # Every run of the same launch gives the same bits: fixed splits and a
    # fixed merge order (the reference pins thread-count invariance bit for
    # bit, tests/sdk/llama_threads.cpp:32-58).
    for r in runs[1:]:
        for i, got in enumerate(r):
            assert np.array_equal(got.view(np.uint32), runs[0][i].view(np.uint32)), f"sequence {i} differs"
    arena.top = mark


# A sequence of at most SHORT_ROWS rows rounds its normalised p to binary16,
# as attend_group does.
SHORT_ROWS = 128


def test_ragged_decode_config4(arena):
    """Config 4 at full size: 16 sequences, lengths U[512, 32768] from the
    seed; the launch runs twice and must give the same bits both times."""
    c = wl.C4
    _ragged(arena, [int(x) for x in c.lengths()], c.n_heads, c.n_kv, c.head_dim, seed=wl.SEED, repeats=2)


def test_ragged_decode_many_short(arena):
    """More sequences than one launch takes (32), lengths from 1 up. Those
    of at most 128 rows take the softmax whole, in a batch with longer ones
    too, and round p where the oracle rounds it."""
    lengths = [1, 2, 31, 32, 33, 128, 129, 500] * 5
    _ragged(arena, lengths, 8, 2, 64, seed=4)


# ---- RoPE ---------------------------------------------------------------------

@pytest.mark.parametrize("mode,yarn,ff", [(0, False, False), (1, False, False), (0, True, False), (0, False, True)])
def test_rope_matches_oracle(arena, mode, yarn, ff):
    hd, heads, n, pos = 128, 4, 9, 4090
    g = wl.rng(17)
    x = wl.normal(g, (n, heads * hd))
    ts = orc.rope_theta_scale(500000.0, hd)
    factors = (1.0 + np.arange(hd // 2) % 4).astype(np.float32) if ff else None
    scaling = [0.25, 1.0, 0.9, 8.0, 23.0] if yarn else None
    mark = arena.top
    in_off = put_rows(arena, x, SYN_F32)
    out_off = arena.alloc(x.nbytes)
    ff_off = put_rows(arena, factors, SYN_F32) if ff else capi.NO_OFFSET
    sc = scaling or [1.0, 0.0, 1.0, 0.0, 0.0]
    d = capi.RopeDesc(in_offset=in_off, out_offset=out_off, freq_factors_offset=ff_off, n=n, size=x.shape[1],
                      head_dim=hd, pos=pos, theta_scale=ts, mode=mode, freq_scale=sc[0], ext_factor=sc[1],
                      attn_factor=sc[2], corr_low=sc[3], corr_high=sc[4])
    check(lib().syn_hip_rope(arena.handle, ctypes.byref(d)))
    got = arena.download(out_off, x.shape, np.float32)
    arena.top = mark
    want = orc.rope_rows(x, hd, pos, ts, freq_factors=factors, mode=mode, scaling=scaling)
    # Same angles bit for bit (repeated f32 multiplication); cos/sin from two
    # libraries, each within an ulp or two.
    assert np.max(np.abs(got - want)) <= 2e-6 * (1 + np.abs(x).max())


def test_rope_position_zero_is_identity(arena):
    x = wl.normal(wl.rng(2), (1, 256))
    in_off = put_rows(arena, x, SYN_F32)
    out_off = arena.alloc(x.nbytes)
    d = capi.RopeDesc(in_offset=in_off, out_offset=out_off, freq_factors_offset=capi.NO_OFFSET, n=1, size=256,
                      head_dim=64, pos=0, theta_scale=orc.rope_theta_scale(1e4, 64), mode=0, freq_scale=1.0,
                      ext_factor=0.0, attn_factor=1.0, corr_low=0.0, corr_high=0.0)
    check(lib().syn_hip_rope(arena.handle, ctypes.byref(d)))
    assert np.array_equal(arena.download(out_off, x.shape, np.float32), x)


def _rope_desc(in_off, out_off, n, size, hd, pos, period=0, mode=0):
    return capi.RopeDesc(in_offset=in_off, out_offset=out_off, freq_factors_offset=capi.NO_OFFSET, n=n, size=size,
                         head_dim=hd, pos=pos, theta_scale=orc.rope_theta_scale(5e5, hd), mode=mode, freq_scale=1.0,
                         ext_factor=0.0, attn_factor=1.0, corr_low=0.0, corr_high=0.0, period=period)


def test_rope_period_restarts_positions_per_image(arena):
    """Several images in one launch (period = rows per image): each image's
    rows are rotated at pos, pos + 1, ... as separate per-image calls do."""
    rows, images, hd, size = 5, 3, 64, 256
    x = wl.normal(wl.rng(8), (rows * images, size))
    mark = arena.top
    in_off = put_rows(arena, x, SYN_F32)
    one, each = arena.alloc(x.nbytes), arena.alloc(x.nbytes)
    check(lib().syn_hip_rope(arena.handle, ctypes.byref(_rope_desc(in_off, one, rows * images, size, hd, 7, rows))))
    for img in range(images):
        at = img * rows * size * 4
        check(lib().syn_hip_rope(arena.handle, ctypes.byref(_rope_desc(in_off + at, each + at, rows, size, hd, 7))))
    got, want = arena.download(one, x.shape, np.float32), arena.download(each, x.shape, np.float32)
    arena.top = mark
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rope_cos_sin_are_correctly_rounded(arena):
    """Rotating (1, 0) pairs returns each pair's (cos, sin): the angle is the
    f32 chain pos * theta_scale^p, and cos and sin of it are the correctly
    rounded f32 values (float64 on the host), for positions up to 2^31."""
    hd = 128
    pos = np.array([0, 1, 4095, 4096, 131071, 2**24 + 1, 2**31 - 5], dtype=np.uint32)
    x = np.tile(np.array([1.0, 0.0], np.float32), hd // 2)[None, :]
    mark = arena.top
    in_off = put_rows(arena, x, SYN_F32)
    out = arena.alloc(x.nbytes)
    ts = np.float32(orc.rope_theta_scale(5e5, hd))
    wrong = 0
    for p in pos:
        check(lib().syn_hip_rope(arena.handle, ctypes.byref(_rope_desc(in_off, out, 1, hd, hd, int(p)))))
        got = arena.download(out, x.shape, np.float32)[0]
        theta = np.empty(hd // 2, np.float32)
        th = np.float32(p)
        for i in range(hd // 2):
            theta[i] = th
            th = np.float32(th * ts)
        cs = np.cos(theta.astype(np.float64)).astype(np.float32)
        sn = np.sin(theta.astype(np.float64)).astype(np.float32)
        wrong += int(np.sum(got[0::2] != cs) + np.sum(got[1::2] != sn))
        assert np.all(np.abs(got[0::2] - cs) <= np.spacing(np.abs(cs))) and \
            np.all(np.abs(got[1::2] - sn) <= np.spacing(np.abs(sn)))
    arena.top = mark
    assert wrong <= 1, wrong  # float64 then float32 may round a rare tie twice


# ---- descriptor checks (nothing is launched) ------------------------------------

def test_bad_descriptors_are_errors_not_faults(arena):
    cache = capi.kv_state(arena, 64, 2, 16)
    base = dict(cache=cache, q_offset=0, k_offset=0, v_offset=0, out_offset=0, scratch_offset=0, scratch_bytes=0,
                n_heads=4, pos=0, n=1, scale=0.25, q_dtype=SYN_F32, kv_dtype=SYN_F32)

    def status(**kw):
        d = capi.AttnDesc(**{**base, **kw})
        return lib().syn_hip_attention(arena.handle, ctypes.byref(d))

    assert status(q_offset=arena.nbytes - 8) == -2       # q outside the arena
    assert status(scale=0.0) == -1                       # bad_parameter
    assert status(scale=float("nan")) == -1
    assert status(n_heads=3) == -1                       # 3 heads on 2 KV heads
    assert status(pos=64) == -1                          # past max_ctx
    assert status(n=0) == -1
    assert status(q_offset=4) == -1                      # misaligned
    bad = capi.KvDesc(k_offset=arena.nbytes, v_offset=0, max_ctx=64, n_kv_heads=2, head_dim=16, ctx_stride=64)
    assert status(cache=bad) == -2
    bad = capi.KvDesc(k_offset=0, v_offset=0, max_ctx=64, n_kv_heads=2, head_dim=258, ctx_stride=64)
    assert status(cache=bad) == -1                       # head_dim > 256
    assert lib().syn_hip_last_error()
