"""Writes the golden fixtures in tests/golden/*.npz.

The fixtures pin the float64 CPU oracle (oracle/dinov3_oracle.c) against an
independent implementation of the same network: the third-party
transformers `DINOv3ViTModel` (not the reference; transformers 5.15.0 as
installed in this image), built from a local config matching ViT-S+/16
(use_gated_mlp, 4 registers, silu, RoPE theta 100), cast to float64, with the
RoPE inverse frequencies and patch coordinates evaluated in float64
(transformers evaluates them in float32), on the seeded random-init weights of dinov3_hrx.write_random_weights.

Each fixture holds the seeds, a per-tensor checksum of the weights it was
made with (so generator drift is caught), the input checksum, and output rows
/ norms of the float64 forward. Run from the repository root:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "dinov3-loom_amd"))
OUT = os.path.dirname(os.path.abspath(__file__))

ROWS = [0, 1, 2, 3, 4, 5, 6, 20]  # prefix rows and the first patches (T >= 21)


def hf_model(grid: int, tensors: dict):
    import torch
    from transformers import DINOv3ViTConfig, DINOv3ViTModel

    cfg = DINOv3ViTConfig(hidden_size=384, intermediate_size=1536, num_hidden_layers=12, num_attention_heads=6,
                          use_gated_mlp=True, num_register_tokens=4, hidden_act="silu", layerscale_value=1.0,
                          layer_norm_eps=1e-5, rope_theta=100.0, image_size=16 * grid, patch_size=16,
                          query_bias=True, key_bias=False, value_bias=True, proj_bias=True, mlp_bias=True)
    model = DINOv3ViTModel(cfg).eval()
    state = {}
    for k, v in tensors.items():
        key = "model." + k if k.startswith("layer.") else k
        state[key] = torch.from_numpy(np.array(v, dtype=np.float64))
    model = model.double()
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected, unexpected
    assert all("inv_freq" in m for m in missing), missing
    head_dim = 64
    inv = 1.0 / (100.0 ** torch.arange(0, 1, 4 / head_dim, dtype=torch.float64))
    model.rope_embeddings.inv_freq = inv
    # transformers evaluates the patch coordinates in float32; evaluate the
    # same expression (its own coordinate helper) in float64 instead.
    from transformers.models.dinov3_vit.modeling_dinov3_vit import get_patches_center_coordinates

    def rope_f64(pixel_values):
        _, _, h, w = pixel_values.shape
        coords = get_patches_center_coordinates(h // 16, w // 16, dtype=torch.float64, device="cpu")
        angles = (2 * math.pi * coords[:, :, None] * inv[None, None, :]).flatten(1, 2).tile(2)
        return torch.cos(angles), torch.sin(angles)

    model.rope_embeddings.forward = rope_f64
    return model


def main() -> None:
    import torch
    from safetensors.numpy import load_file

    import dinov3_hrx as d

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    names = oracle.tensor_names()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    cases = [
        ("g4_baseline", 4, 0, "full"),
        ("g4_stress", 4, 1, "full"),
        ("g14_baseline", 14, 0, "rows"),
        ("g14_stress", 14, 1, "rows"),
        ("g32_stress", 32, 1, "rows"),
    ]
    with tempfile.TemporaryDirectory() as tmp:
        for preset in (0, 1):
            path = os.path.join(tmp, f"w{preset}.safetensors")
            d.write_random_weights(path, seed=0, preset=preset)
        for name, grid, preset, kind in cases:
            tensors = load_file(os.path.join(tmp, f"w{preset}.safetensors"))
            pixels = d.random_pixels(1, 1, 16 * grid)
            model = hf_model(grid, tensors)
            with torch.no_grad():
                out = model(pixel_values=torch.from_numpy(pixels.astype(np.float64))).last_hidden_state[0].numpy()
            T = grid * grid + 5
            assert out.shape == (T, 384)
            rec = {
                "grid": np.int64(grid), "preset": np.int64(preset), "weight_seed": np.int64(0),
                "pixel_seed": np.int64(1),
                "weight_sums": np.array([np.sum(np.asarray(tensors[n], np.float64)) for n in names]),
                "pixel_sum": np.float64(np.sum(pixels.astype(np.float64))),
                "norms": np.linalg.norm(out, axis=1),
                "total": np.float64(out.sum()),
            }
            if kind == "full":
                rec["out"] = out
            else:
                rec["rows"] = np.array(ROWS + [T - 1], np.int64)
                rec["row_values"] = out[ROWS + [T - 1]]
            np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **rec)
            print(name, out.shape, float(out.std()))
        # RoPE tables as transformers builds them (float64 angles, stored f32).
        for grid in (14, 32):
            from transformers.models.dinov3_vit.modeling_dinov3_vit import get_patches_center_coordinates
            coords = get_patches_center_coordinates(grid, grid, dtype=torch.float64, device="cpu")
            inv = 1.0 / (100.0 ** torch.arange(0, 1, 4 / 64, dtype=torch.float64))
            angles = 2 * math.pi * coords[:, :, None] * inv[None, None, :]
            angles = angles.flatten(1, 2).tile(2)
            np.savez_compressed(os.path.join(OUT, f"rope_g{grid}.npz"), cos=torch.cos(angles).numpy().astype(np.float32),
                                sin=torch.sin(angles).numpy().astype(np.float32))


if __name__ == "__main__":
    main()
