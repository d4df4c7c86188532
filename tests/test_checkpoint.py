"""The synthetic checkpoint writer (qwen_wlqfastshot_helen_beta_amd/checkpoint.py) on a small
model: the tensors the plugin's create_weights registers, in the reference's on-disk dtypes
and shapes (vllm_wlq/linear_method.py:376-411), EF tiles that decode (oracle decoder) to as
many positions as there are outlier values, and the adapter directory get_dora_adapter
reads (vllm_wlq/linear_method.py:17-120)."""
from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import checkpoint as C
from qwen_wlqfastshot_helen_beta_amd import formats

SMALL = C.ModelDims(hidden=256, intermediate=640, kv=64, layers=2)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    path = tmp_path_factory.mktemp("ckpt")
    C.write_synthetic_checkpoint(str(path), SMALL, bits=4, density=0.01, rank=8, lora_alpha=16, tile_size=32, seed=1)
    return path


def test_checkpoint_tensors(ckpt):
    import torch
    from safetensors import safe_open

    projs = C._projections(SMALL)
    for l in range(SMALL.layers):
        with safe_open(str(ckpt / f"model-{l:05d}.safetensors"), framework="pt", device="cpu") as f:
            keys = set(f.keys())
            assert len(keys) == 7 * 7
            for p, (mod, N, K) in projs.items():
                pre = f"model.layers.{l}.{mod}.{p}"
                q = f.get_tensor(f"{pre}.q_packed")
                assert q.dtype == torch.int32 and q.numel() == -(-N * K // 8)
                codes = O.unpack_continuous(q.numpy().view(np.uint32), N, K, 4)
                assert codes.max() <= 15 and len(np.unique(codes)) == 16
                lut = f.get_tensor(f"{pre}.lut_c")
                assert lut.dtype == torch.float16 and tuple(lut.shape) == (N, 16)
                assert np.all(np.diff(lut.numpy().astype(np.float32), axis=1) >= 0)  # sorted LUTs
                assert int(f.get_tensor(f"{pre}.bits").item()) == 4
                T = int(f.get_tensor(f"{pre}.ef_tile_size").item())
                meta = f.get_tensor(f"{pre}.ef_tile_meta").numpy()
                bs = f.get_tensor(f"{pre}.ef_bitstream").numpy().view(np.uint32)
                vals = f.get_tensor(f"{pre}.outlier_values")
                assert meta.dtype == np.int64 and vals.dtype == torch.float8_e5m2
                mask = O.ef_decode_mask(meta, bs, N, K, T)
                assert int(mask.sum()) == vals.numel() > 0
                assert abs(mask.mean() - 0.01) < 0.005
    a = json.loads((ckpt / "lora_adapter_distilled" / "adapter_config.json").read_text())
    assert a["r"] == 8 and a["lora_alpha"] == 16
    with safe_open(str(ckpt / "lora_adapter_distilled" / "adapter_model.safetensors"), framework="pt",
                   device="cpu") as f:
        A = f.get_tensor("base_model.model.model.layers.1.mlp.down_proj.lora_A.weight")
        B = f.get_tensor("base_model.model.model.layers.1.mlp.down_proj.lora_B.weight")
        assert tuple(A.shape) == (8, SMALL.intermediate) and tuple(B.shape) == (SMALL.hidden, 8)


def test_random_codes_tail_is_zero():
    rng = np.random.default_rng(0)
    for bits, N, K in ((4, 3, 5), (3, 7, 9), (4, 16, 64)):
        w = C._random_codes_continuous(rng, N, K, bits)
        spw = formats.symbols_per_word(bits)
        assert w.size == -(-N * K // spw)
        codes = O.unpack_continuous(w, N, K, bits)
        assert codes.max() < (1 << bits)
        tail = N * K - (w.size - 1) * spw
        assert int(w[-1]) >> (tail * bits) == 0
