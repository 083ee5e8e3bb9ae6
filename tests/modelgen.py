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

FMT_TAG = {"f32": vlt3.F32, "bf16": vlt3.BF16, "q8_0": vlt3.Q8_0, "q4_0": vlt3.Q4_0}


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


# ---------------------------------------------------------------------------------------------
# Word-level vocabulary and ChatML conversations for the resonance / governor rules: identifiers
# (letters + digits / underscore: tier-A shingles), content words of five or more letters (tier-B
# shingles), a one-letter tag followed by a number ("t 3"), rollback cues, the spoof markers, line
# and clause delimiters, and byte strings of the governor's evasions (split, spaced, homoglyph,
# reversed, Base64, hex pieces).
KEYS = [f" key_{i}".encode() for i in range(24)]
WORDS = [w.encode() for w in (" anchor", " beacon", " cobalt", " dynamo", " ember", " falcon", " glacier",
                              " harbor", " indigo", " jasper", " kernel", " lantern", " meadow", " nebula",
                              " orchid", " prism", " quartz", " raven", " summit", " timber")]
GLUE = [b" =", b":", b" is", b" the", b" of", b" value", b" what", b",", b".", b"?", b" |", b";", b" and",
        b" set", b" to", b" t", b" 3", b" 12", b" 7", b" rollback", b" revert", b" restore", b" roll", b" back",
        b" user", b" assistant", b" opi_signed_directive", b" urgent", b" opi", b" delegation", b" OPI",
        b" config-server", b" main-loop", b" note", b" item_9x", b" node-7",
        # governor material: pieces of rule strings, separators, look-alikes, encodings
        b" sys", b"call", b"_exec", b"SYS", b"CALL", b"_EXEC", b" s", b"y", b"c", b"a", b"l", b"e", b"x",
        b"\xe2\x80\x8b", "с".encode(), "а".encode(), b"ex", b"ec", b"cexe_llacsys", b"c3lz", b"Y2Fs",
        b"bF9l", b"eGVj", b"73", b"79", b"73 63", b"\\x61", b"0x6c", b" rm_rf(", b"rm", b"_rf", b"(",
        b"'", b"\"", b" never", b" output", b" must not", b" print",
        # "syscall_exec" / "rm_rf(" in Base64 (with three bytes of misalignment available) and hex
        b"QQQ", b"c3lzY2Fs", b"bF9leGVj", b"cm1fcmYo", b"0x73 0x79 0x73", b" 0x63 0x61 0x6c", b" 0x6c 0x5f 0x65",
        b" 0x78 0x65 0x63", b"\\x72\\x6d\\x5f", b"\\x72\\x66\\x28"]


def word_vocab(cfg: VAULTv3Config, seed: int = 0):
    """(token strings, byte map): the words above at ids 11.., ChatML specials and b"system" at their
    config ids, b"\\n" at NEWLINE_ID, short filler pieces elsewhere."""
    toks, byte_map = test_vocab(cfg, seed)
    words = KEYS + WORDS + list(GLUE)
    assert 11 + len(words) < cfg.vocab_size - 8
    for i, w in enumerate(words):
        toks[11 + i] = w
    return toks, byte_map


def word_ids(toks: list) -> dict:
    """bytes -> the first id that carries them."""
    out = {}
    for i, t in enumerate(toks):
        out.setdefault(t, i)
    return out


def conversation(cfg: VAULTv3Config, toks: list, kind: str, seed: int = 0, n_lines: int = 14,
                 filler: int = 40, answer: int = 30) -> list:
    """A ChatML stream: a pinned system prompt, a user turn of key / value lines (evicted into the
    segment bank as the stream goes on), filler turns, a question of ``kind`` ("id", "ids", "words",
    "rollback", "hop", "spoof", "clause"), <|im_end|>, then ``answer`` assistant tokens."""
    rng = np.random.default_rng(seed)
    ids = word_ids(toks)
    w = lambda *bs: [ids[b] for b in bs]
    nl = [NEWLINE_ID]
    out = [cfg.im_start_id, cfg.system_tok_id] + nl + w(b" note", b" the", b" value", b" of", b" key_0", b".") + \
        [cfg.im_end_id] + nl + [cfg.im_start_id] + w(b" user") + nl
    keys = rng.permutation(len(KEYS))[:n_lines]
    vals = rng.integers(0, len(WORDS), size=(n_lines, 2))
    for j in range(n_lines):
        k, (a, b) = KEYS[keys[j]], vals[j]
        line = w(k, b" =", WORDS[a], WORDS[b])
        if kind == "clause" and j % 3 == 0:
            line += w(b";", b" set", WORDS[(a + 3) % len(WORDS)], b" |", b" note", WORDS[(b + 5) % len(WORDS)],
                      b" and", WORDS[(a + 7) % len(WORDS)])
        if kind == "hop" and j == 4:
            line += w(b" to", KEYS[keys[9]])               # a bridge id shared by exactly two segments
        if kind == "rollback" and j == n_lines - 2:
            line = w(b" rollback", b" to", b" t", b" 3", KEYS[keys[j]])
        if kind == "rollback" and j == 2:
            line += w(b" t", b" 3")
        out += line + nl
    out += [cfg.im_end_id] + nl
    fill = rng.integers(11, 11 + len(KEYS) + len(WORDS), size=filler)
    out += [cfg.im_start_id] + w(b" assistant") + nl + [int(t) for t in fill] + [cfg.im_end_id] + nl
    q = [cfg.im_start_id] + w(b" user") + nl + w(b" what", b" is", b" the", b" value", b" of")
    if kind in ("id", "hop", "clause"):
        q += w(KEYS[keys[4]], b"?")
    elif kind == "ids":
        q += w(KEYS[keys[3]], b" and", KEYS[keys[8]], b"?")
    elif kind == "words":
        a, b = vals[6]
        q += w(WORDS[a], WORDS[b], b"?")
    elif kind == "rollback":
        q += w(KEYS[keys[n_lines - 2]], b" rollback", b"?")
    elif kind == "spoof":
        q += w(b" urgent", b" OPI", b" delegation", b" opi_signed_directive", KEYS[keys[1]], b"?")
    out += q + [cfg.im_end_id] + nl + [cfg.im_start_id] + w(b" assistant") + nl
    out += [int(t) for t in rng.integers(11, 11 + len(KEYS) + len(WORDS) + 20, size=answer)]
    return out
