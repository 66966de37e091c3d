"""Runs the C++20 host tests (tests/cpp/, built by python -m synapse_amd.build):
the graph builder and planner on the CPU, the session through the C ABI on
the GPU against the CPU oracle."""
from __future__ import annotations

import pathlib
import subprocess

import pytest

BIN = pathlib.Path(__file__).resolve().parent / "cpp" / "_bin"
DATA = pathlib.Path(__file__).resolve().parent / "golden" / "reference"


def _run(name: str, *args: str) -> None:
    exe = BIN / name
    if not exe.exists():
        pytest.fail(f"{exe} is missing: build with `python -m synapse_amd.build`")
    proc = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=300)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def _dump_model(name: str, out: pathlib.Path) -> None:
    """Writes a reference fixture's weights (as the file stores them), its
    config, tokens and golden logits where test_model_session reads them."""
    import numpy as np

    from synapse_amd.gguf import GGUFFile
    from synapse_amd.llama import _f32_weight, _matrix, read_config

    model = GGUFFile(DATA / f"{name}.gguf")
    golden = GGUFFile(DATA / f"{name}_golden.gguf")
    c = read_config(model)
    hd, q_rows, kv_rows = c.head_dim, c.n_head * c.head_dim, c.n_head_kv * c.head_dim
    shapes = {"token_embd.weight": (c.n_vocab, c.n_embd), "output_norm.weight": (1, c.n_embd),
              "output.weight": (c.n_vocab, c.n_embd), "output.bias": (1, c.n_vocab), "rope_freqs.weight": (1, hd // 2)}
    for l in range(c.n_layer):
        p = f"blk.{l}."
        shapes.update({p + "attn_norm.weight": (1, c.n_embd), p + "ffn_norm.weight": (1, c.n_embd),
                       p + "attn_q.weight": (q_rows, c.n_embd), p + "attn_k.weight": (kv_rows, c.n_embd),
                       p + "attn_v.weight": (kv_rows, c.n_embd), p + "attn_output.weight": (c.n_embd, q_rows),
                       p + "ffn_gate.weight": (c.n_ff, c.n_embd), p + "ffn_up.weight": (c.n_ff, c.n_embd),
                       p + "ffn_down.weight": (c.n_embd, c.n_ff), p + "attn_q.bias": (1, q_rows),
                       p + "attn_k.bias": (1, kv_rows), p + "attn_v.bias": (1, kv_rows),
                       p + "attn_output.bias": (1, c.n_embd), p + "ffn_gate.bias": (1, c.n_ff),
                       p + "ffn_up.bias": (1, c.n_ff), p + "ffn_down.bias": (1, c.n_embd)})
    blob, lines = bytearray(), []
    for tname, (rows, cols) in shapes.items():
        if tname not in model.tensors:
            continue
        if rows == 1:  # norms, biases, RoPE factors: F32 vectors
            t, data = 0, _f32_weight(model, tname, (cols,))
        else:
            t, data = _matrix(model, tname, rows, cols)
        raw = np.ascontiguousarray(data).tobytes()
        lines.append(f"{tname} {t} {rows} {cols} {len(blob)} {len(raw)}")
        blob += raw + bytes(-len(raw) % 64)
    (out / "weights.bin").write_bytes(bytes(blob))
    (out / "manifest.txt").write_text("\n".join(lines) + "\n")
    f32 = lambda x: repr(float(np.float32(x)))
    s = c.rope_scaling
    cfg = {"n_layer": c.n_layer, "n_embd": c.n_embd, "n_head": c.n_head, "n_head_kv": c.n_head_kv, "head_dim": hd,
           "n_vocab": c.n_vocab, "rope_mode": c.rope_mode, "n_ctx_orig": c.n_ctx_orig, "rms_eps": f32(c.rms_eps),
           "rope_base": f32(c.rope_base), "attn_temp_scale": f32(c.attn_temp_scale), "freq_scale": f32(s.freq_scale),
           "ext_factor": f32(s.ext_factor), "attn_factor": f32(s.attn_factor), "corr_low": f32(s.corr_low),
           "corr_high": f32(s.corr_high)}
    (out / "config.txt").write_text("".join(f"{k} {v}\n" for k, v in cfg.items()))
    tokens = [int(t) for t in golden.require("synapse.golden.tokens")]
    (out / "tokens.txt").write_text(" ".join(map(str, tokens)) + "\n")
    (out / "logits.bin").write_bytes(np.ascontiguousarray(golden.tensor("logits"), dtype=np.float32).tobytes())


def test_graph_builder_and_planner():
    _run("test_graph")


def test_rope_sin_cos_correctly_rounded():
    """The RoPE kernels' own sin and cos (Cody-Waite and Taylor series in
    double), built for the host: correctly rounded for angles up to 2^32."""
    _run("test_rope_math")


def test_session_run_allocates_nothing():
    """session::run under a counting operator new, against a C ABI that
    launches nothing (tests/sdk/graph_no_alloc.cpp:199-263 restated)."""
    _run("test_no_alloc")


@pytest.mark.gpu
def test_session_against_the_oracle():
    _run("test_session")


# The F32 fixtures at the reference's bound (max |ours - ref| / max |ref|
# < 1e-4 and the same argmax, tests/sdk/llama_golden.cpp:80); the quantized
# ones at its rel rms bounds (tests/sdk/llama_golden.cpp:58-73).
MODEL_BOUNDS = {"llama_tiny_f32": ("max", "1e-4"), "qwen2_tiny_f32": ("max", "1e-4"),
                "mistral3_tiny_f32": ("max", "1e-4"), "llama_tiny": ("rms", "2e-2"), "qwen2_tiny": ("rms", "2e-2"),
                "mistral3_tiny": ("rms", "5e-2")}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(MODEL_BOUNDS))
def test_model_graph_through_the_session(tmp_path, name):
    """Every op of a Llama-family graph through graph_builder and session,
    against llama.cpp's logits for the reference's tiny models."""
    _dump_model(name, tmp_path)
    _run("test_model_session", str(tmp_path), *MODEL_BOUNDS[name])


def _dump_clip(out: pathlib.Path) -> None:
    """clip_tiny's weights under the names test_model_session reads, its
    unfolded image and golden embeddings (the projector file's up/down pair
    taken in whichever order it is stored, S/models/clip.hpp:318-323)."""
    import numpy as np

    from synapse_amd.clip import read_config, unfold_patches
    from synapse_amd.gguf import GGUFFile

    model = GGUFFile(DATA / "clip_tiny.gguf")
    golden = GGUFFile(DATA / "clip_tiny_golden.gguf")
    c = read_config(model)
    E, F = c.n_embd, c.n_ff
    names = {"patch.w": "v.patch_embd.weight", "patch.b": "v.patch_embd.bias", "pos": "v.position_embd.weight",
             "post.w": "v.post_ln.weight", "post.b": "v.post_ln.bias", "fc": "mm.model.fc.weight"}
    for l in range(c.n_layer):
        b = f"v.blk.{l}."
        for s in ("ln1.weight", "ln1.bias", "attn_q.weight", "attn_q.bias", "attn_k.weight", "attn_k.bias",
                  "attn_v.weight", "attn_v.bias", "attn_out.weight", "attn_out.bias", "ln2.weight", "ln2.bias"):
            names[b + s] = b + s
        up, down = ("ffn_down", "ffn_up") if model.tensors[b + "ffn_down.weight"].shape[0] == E else ("ffn_up",
                                                                                                      "ffn_down")
        names.update({b + "up.w": b + up + ".weight", b + "up.b": b + up + ".bias", b + "down.w": b + down + ".weight",
                      b + "down.b": b + down + ".bias"})
    blob, lines = bytearray(), []
    for key, tname in names.items():
        if tname not in model.tensors:
            continue
        a = np.ascontiguousarray(model.tensor(tname), dtype=np.float32)
        a = a.reshape(1, -1) if a.ndim == 1 else a.reshape(a.shape[0], -1)  # the patch kernel: (channel, y, x)
        rows, cols = a.shape
        raw = a.tobytes()
        lines.append(f"{key} 0 {rows} {cols} {len(blob)} {len(raw)}")
        blob += raw + bytes(-len(raw) % 64)
    (out / "weights.bin").write_bytes(bytes(blob))
    (out / "manifest.txt").write_text("\n".join(lines) + "\n")
    cfg = {"model": "clip", "n_layer": c.n_layer, "n_embd": E, "n_head": c.n_head, "n_ff": F,
           "eps": repr(float(np.float32(c.eps))), "patch_floats": c.patch_floats, "n_patches": c.n_patches,
           "grid": c.grid, "scale_factor": c.scale_factor, "n_tokens": c.n_tokens, "n_embd_text": c.n_embd_text}
    (out / "config.txt").write_text("".join(f"{k} {v}\n" for k, v in cfg.items()))
    image = np.asarray(golden.tensor("image"), np.float32)
    (out / "patches.bin").write_bytes(np.ascontiguousarray(unfold_patches(c, image), np.float32).tobytes())
    (out / "logits.bin").write_bytes(np.ascontiguousarray(golden.tensor("embeddings"), np.float32).tobytes())


@pytest.mark.gpu
def test_image_encoder_graph_through_the_session(tmp_path):
    """layer_norm, gelu, add_rows, self_attention and pixel_shuffle through
    graph_builder and session against clip_tiny's golden embeddings, at the
    reference's bound (per-token rel rms < 1e-4, tests/sdk/clip_golden.cpp:33)."""
    _dump_clip(tmp_path)
    _run("test_model_session", str(tmp_path), "rowrms", "1e-4")
