"""The C ABI without a GPU: libsynapse_hip.so loads, exports every function
include/synapse_hip.h declares (and the ctypes table binds exactly those),
and its host-only functions -- sizing, error strings, argument checks that
fail before any device work -- behave as documented."""
from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from synapse_amd import capi

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "synapse_hip.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(syn_hip_\w+)\s*\(", text))


def test_header_declares_the_boundary():
    names = _declared()
    for must in ("syn_hip_arena_create", "syn_hip_attention", "syn_hip_attend", "syn_hip_kv_append",
                 "syn_hip_self_attention", "syn_hip_attend_batch", "syn_hip_rope"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_binds_exactly_the_header():
    assert set(capi.SIGNATURES) == _declared()


def test_descriptor_layouts_match_the_header(tmp_path):
    """Compiles the header with the host C compiler and compares every
    descriptor's size and field offsets with the ctypes mirror."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    structs = {"syn_kv_desc": capi.KvDesc, "syn_attn_desc": capi.AttnDesc, "syn_seq_desc": capi.SeqDesc,
               "syn_self_desc": capi.SelfDesc, "syn_rope_desc": capi.RopeDesc, "syn_embed_desc": capi.EmbedDesc,
               "syn_norm_desc": capi.NormDesc, "syn_matmul_desc": capi.MatmulDesc,
               "syn_elementwise_desc": capi.ElementwiseDesc, "syn_layer_norm_desc": capi.LayerNormDesc,
               "syn_pixel_shuffle_desc": capi.PixelShuffleDesc, "syn_matmul_q_desc": capi.MatmulQDesc,
               "syn_softmax_desc": capi.SoftmaxDesc}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, ct in structs.items():
        lines.append(f'printf("{cname} @sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in ct._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c11", "-o", str(exe), str(src)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                          text=True).stdout.splitlines())
    for cname, ct in structs.items():
        assert int(got[f"{cname} @sizeof"]) == ctypes.sizeof(ct), cname
        for fname, _ in ct._fields_:
            assert int(got[f"{cname} {fname}"]) == getattr(ct, fname).offset, (cname, fname)


def test_error_strings():
    lib = capi.lib()
    for code, text in [(0, b"ok"), (-1, b"invalid argument"), (-2, b"offset outside the arena"),
                       (-3, b"unsupported shape"), (-4, b"device allocation failed"), (-5, b"no gfx950 device"),
                       (-99, b"unknown error")]:
        assert lib.syn_hip_error_string(code) == text


@pytest.mark.parametrize("max_ctx,stride", [(1, 64), (64, 64), (65, 128), (4097, 4160), (32768, 32768)])
def test_kv_ctx_stride(max_ctx, stride):
    assert capi.lib().syn_hip_kv_ctx_stride(max_ctx) == stride


def test_kv_state_bytes():
    lib = capi.lib()
    # config 2: K 4097 rows x 2 KiB (256-aligned) then V^T 1024 rows x 4160 halves
    k = (4097 * 1024 * 2 + 255) // 256 * 256
    assert lib.syn_hip_kv_state_bytes(4097, 8, 128) == k + 1024 * 4160 * 2
    # never smaller than the reference's unpadded state_desc::bytes (2*2*max_ctx*n_kv*hd)
    for shape in [(12, 2, 16), (33, 3, 40), (1, 1, 2)]:
        assert lib.syn_hip_kv_state_bytes(*shape) >= 4 * shape[0] * shape[1] * shape[2]


def test_attention_scratch_bytes():
    lib = capi.lib()
    # split-KV partials: ceil(max_ctx / 128) splits x n_kv x group x (hd + 2) floats
    want = ((4097 + 127) // 128) * 8 * 4 * (128 + 2) * 4
    assert lib.syn_hip_attention_scratch_bytes(32, 8, 128, 4097, 1) == (want + 255) // 256 * 256
    assert lib.syn_hip_attention_scratch_bytes(30, 8, 128, 4097, 1) == 0  # heads not a multiple of n_kv


def test_null_arguments_are_errors():
    lib = capi.lib()
    assert lib.syn_hip_arena_create(1024, None) == -1
    assert lib.syn_hip_arena_destroy(None) == 0
    assert lib.syn_hip_arena_bytes(None) == 0
    assert lib.syn_hip_arena_stream(None) is None
    assert lib.syn_hip_synchronize(None) == -1
    assert lib.syn_hip_upload(None, 0, None, 0) == -1
    d = capi.AttnDesc()
    assert lib.syn_hip_attention(None, ctypes.byref(d)) == -1
    assert lib.syn_hip_attend(None, ctypes.byref(d)) == -1
    assert lib.syn_hip_self_attention(None, None) == -1
    assert lib.syn_hip_rope(None, None) == -1
    assert b"null" in lib.syn_hip_last_error()
