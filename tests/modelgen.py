"""Tiny seeded models shared by the tests: config, fp32 state, quantized tensors, a VLT3 image, and
the dequantized weights the oracle consumes."""
from __future__ import annotations

import os
import tempfile

import numpy as np

from oracle import codec
from vault_amd import vlt3
from vault_amd.config import VAULTv3Config
from vault_amd.tokens import build_vtok
from vault_amd.weights import quantize_state, random_state

FMT_TAG = {"f32": vlt3.F32, "q8_0": vlt3.Q8_0, "q4_0": vlt3.Q4_0}


def tiny_cfg(head_dim=64, n_layers=2, window=16, seg_budget=12, vocab=2048, n_heads=4, n_kv_heads=2,
             **kw) -> VAULTv3Config:
    H, G = n_heads, n_kv_heads
    d = H * head_dim
    base = dict(vocab_size=vocab, d_model=d, n_layers=n_layers, n_heads=H, n_kv_heads=G, head_dim=head_dim,
                d_ff=2 * d, window=window, n_sink=4, max_sink=8, rope_theta=1_000_000.0,
                im_start_id=vocab - 4, im_end_id=vocab - 3, system_tok_id=vocab - 2,
                seg_budget=seg_budget, seg_hidden=32, seg_min=3, seg_max=7,
                seg_layers=(0, 1) if seg_budget > 0 else ())
    base.update(kw)
    return VAULTv3Config(**base)


# Token strings of the test vocabulary: short space-led words (at most four letters, so the C
# runtime's shingle extractor finds nothing and its resonance bias stays off), white space and the
# delimiters of every segment-break tier.
_PIECES = [b" ab", b" cd.", b"}", b",", b" efg", b"!", b"\t", b" hi;", b"", b'",', b" jk ", b"&", b"?  ",
           b" lm", b"]", b" no|", b" pq\n", b" rs", b" tu", b" vw", b"\r\n", b" xy", b" z", b"; "]
NEWLINE_ID = 10


def test_vocab(cfg: VAULTv3Config, seed: int = 0):
    """(token strings, byte map) of a tiny model: ChatML specials at their config ids, b"system" at
    cfg.system_tok_id, b"\n" at NEWLINE_ID (the byte map's entry for '\n'; not 198, so the byte rule
    and the Python rule differ), and the pieces above drawn with a seeded generator elsewhere."""
    rng = np.random.default_rng(seed)
    toks = [_PIECES[i] for i in rng.integers(0, len(_PIECES), size=cfg.vocab_size)]
    toks[cfg.im_start_id] = b"<|im_start|>"
    toks[cfg.im_end_id] = b"<|im_end|>"
    toks[cfg.system_tok_id] = b"system"
    toks[NEWLINE_ID] = b"\n"
    byte_map = [0] * 256
    byte_map[0x0A] = NEWLINE_ID
    return toks, byte_map


def build(cfg: VAULTv3Config, fmt: str, seed: int = 3, vocab=None):
    """Seeded tensors, the VLT3 image of them (with the VTOK of ``vocab`` = (token strings, byte map)
    when given, else empty token strings) and the dequantized weights the oracle consumes."""
    state = random_state(cfg, seed)
    tensors = quantize_state(cfg, state, fmt)
    blob = build_vtok(vocab[0], vocab[1]) if vocab is not None else None
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.vlt3")
        vlt3.write_vlt3(path, list(tensors.values()), cfg, FMT_TAG[fmt], tok_blob=blob)
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
    """Ordinary token ids (below vocab - 8: never a ChatML special or the system-role token)."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, cfg.vocab_size - 8, size=n).tolist()


def chatml_prefix(cfg: VAULTv3Config, sys_len: int, nl_after_end: bool = True, system: bool = True) -> list:
    """<|im_start|> system \n, sys_len ordinary ids, <|im_end|>, then \n when nl_after_end."""
    rng = np.random.default_rng(1000 + sys_len)
    body = [int(t) for t in rng.integers(11, cfg.vocab_size - 8, size=sys_len)]
    head = [cfg.im_start_id] + ([cfg.system_tok_id, NEWLINE_ID] if system else [11])
    return head + body + [cfg.im_end_id] + ([NEWLINE_ID] if nl_after_end else [])
