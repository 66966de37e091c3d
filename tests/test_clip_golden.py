"""The reference's image-encoder fixture: a tiny random-weight idefics3
mmproj (SigLIP ViT with 4 heads of 16 over 64 patches, pixel shuffle,
linear projector; F32 matrices) and the embeddings llama.cpp's clip.cpp
computes for a fixed image (tests/data/README.md of the reference). The
reference's bound is rms(ours - ref) / rms(ref) < 1e-4 per output token
(tests/sdk/clip_golden.cpp:22-35).

test_cpu_*: this build's reading of the graph on the CPU oracle (f32
self-attention, as the reference computes it), at the reference's bound.
test_gpu_*: the whole encoder on the device through the C ABI, at the same
bound: f32 image rows take the device's f32 self-attention, whose fma chains
follow the reference's order (S/kernels/attention.hpp:324-486). A wrong op
or layout moves the embeddings by O(1)."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

from clip_host import compare, encode
from synapse_amd.clip import read_config, unfold_patches
from synapse_amd.gguf import GGUFFile

DATA = pathlib.Path(__file__).resolve().parent / "golden" / "reference"
BOUND = 1e-4


def _load():
    model = GGUFFile(DATA / "clip_tiny.gguf")
    golden = GGUFFile(DATA / "clip_tiny_golden.gguf")
    return model, np.asarray(golden.tensor("image"), np.float32), np.asarray(golden.tensor("embeddings"), np.float32)


def test_clip_config_and_unfold():
    model, image, ref = _load()
    c = read_config(model)
    assert (c.image_size, c.patch_size, c.n_embd, c.n_head, c.n_layer, c.scale_factor, c.n_embd_text) == \
        (64, 8, 64, 4, 2, 2, 48)
    assert ref.shape == (c.n_tokens, c.n_embd_text) == (16, 48)
    p = unfold_patches(c, image)
    img = image.reshape(64, 64, 3)
    # patch (px=2, py=1), channel 1, pixel (y=3, x=5) of the patch
    assert p[2 + 8 * 1, (1 * 8 + 3) * 8 + 5] == img[1 * 8 + 3, 2 * 8 + 5, 1]


def test_cpu_encode_matches_llama_cpp():
    model, image, ref = _load()
    errs = compare(encode(model, image), ref)
    assert max(errs) < BOUND, errs


@pytest.mark.gpu
def test_gpu_encode_matches_llama_cpp():
    from synapse_amd.clip import DeviceClip
    model, image, ref = _load()
    m = DeviceClip(model)
    try:
        got = m.encode(image)
    finally:
        m.close()
    errs = compare(got, ref)
    assert max(errs) < BOUND, errs
