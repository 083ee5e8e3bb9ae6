"""Tiny seeded models shared by the tests: config, fp32 state, quantized tensors, a VLT3 image, and
the dequantized weights the oracle consumes."""
from __future__ import annotations

import os
import tempfile

import numpy as np

from oracle import codec
from vault_amd import vlt3
from vault_amd.config import VAULTv3Config
from vault_amd.weights import quantize_state, random_state

FMT_TAG = {"f32": vlt3.F32, "q8_0": vlt3.Q8_0, "q4_0": vlt3.Q4_0}


def tiny_cfg(head_dim=64, n_layers=2, window=16, seg_budget=12, vocab=2048, **kw) -> VAULTv3Config:
    H, G = 4, 2
    d = H * head_dim
    base = dict(vocab_size=vocab, d_model=d, n_layers=n_layers, n_heads=H, n_kv_heads=G, head_dim=head_dim,
                d_ff=2 * d, window=window, n_sink=4, max_sink=8, rope_theta=1_000_000.0,
                im_start_id=vocab - 4, im_end_id=vocab - 3, system_tok_id=vocab - 2,
                seg_budget=seg_budget, seg_hidden=32, seg_min=3, seg_max=7,
                seg_layers=(0, 1) if seg_budget > 0 else ())
    base.update(kw)
    return VAULTv3Config(**base)


def build(cfg: VAULTv3Config, fmt: str, seed: int = 3):
    state = random_state(cfg, seed)
    tensors = quantize_state(cfg, state, fmt)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.vlt3")
        vlt3.write_vlt3(path, list(tensors.values()), cfg, FMT_TAG[fmt])
        with open(path, "rb") as f:
            image = f.read()
    deq = {}
    for name, t in tensors.items():
        rows = t.shape[0] if len(t.shape) == 2 else 1
        cols = t.shape[-1]
        a = codec.decode(t.dtype, t.data, rows, cols)
        deq[name] = a.reshape(t.shape)
    return tensors, image, deq


def ids_stream(cfg: VAULTv3Config, n: int, seed: int = 0) -> list:
    rng = np.random.default_rng(seed)
    return rng.integers(0, cfg.vocab_size - 8, size=n).tolist()
