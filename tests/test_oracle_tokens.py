"""Token-byte rules (segment-break tiers, system role, newline id, VTOK parsing) and the auto-pin
state machine, pinned against the reference C runtime (runtime/vault3.c compiled into oracle/_ref)
on models whose VLT3 files carry real token strings.

Bars: the tier function of the product equals the oracle's restatement on every byte string of a
small alphabet (brute force) and the C runtime's own comments (runtime/vault3.c:933-936) as known
answers; the oracle model against the C runtime: n_pin, pin_locked and the segment-memory slots
exactly, logits rel < 1e-4 with 100% top-1 (tests/test_vlt3_runtime.py:90-94), and the C runtime's
resonance bias never active (the test vocabulary holds no shingle-forming words).
"""
import itertools

import numpy as np
import pytest

from oracle import ref
from oracle import tokens as otok
from oracle.model import OracleModel
from tests import modelgen
from vault_amd import tokens as vtok


@pytest.mark.parametrize("b,want", [
    (b"\n", 1), (b" end.", 1), (b"ok!  \t", 1), (b"why?\r", 1), (b"a;", 1), (b"x\ny,", 1),
    (b"}", 2), (b"]", 2), (b" a|b", 2), (b"\t", 2), (b'"k",', 2), (b"a}.", 1),
    (b",", 3), (b"a&b", 3), (b" x,", 3), (b'",', 2),
    (b"", 0), (b" ab", 0), (b".x", 0), (b"(", 0), (b"\r", 0),
])
def test_break_tier_known_answers(b, want):
    assert vtok.break_tier(b) == want
    assert otok.tier(b) == want


def test_break_tier_brute_force():
    alpha = b' \t\r\n.,!?;}]|"&a\x0b\x0c'
    for n in range(4):
        for t in itertools.product(alpha, repeat=n):
            b = bytes(t)
            assert vtok.break_tier(b) == otok.tier(b), b


def test_vtok_round_trip_and_rules():
    cfg = modelgen.tiny_cfg()
    toks, bmap = modelgen.test_vocab(cfg)
    tt = vtok.TokenTable.from_vtok(vtok.build_vtok(toks, bmap), cfg.vocab_size)
    assert tt.tokens == toks and tt.newline_id == modelgen.NEWLINE_ID
    assert tt.is_system_role(cfg.system_tok_id) and not tt.is_system_role(cfg.im_start_id)
    assert vtok.TokenTable([b"system\n"], [0] * 256, 4).is_system_role(0)
    assert not vtok.TokenTable([b"systems"], [0] * 256, 4).is_system_role(0)
    assert [int(x) for x in tt.tiers] == [otok.tier(b) for b in toks]
    assert not tt.is_system_role(cfg.vocab_size + 5) and tt.bytes_of(-1) == b""


def test_vtok_rejects_malformed_blobs():
    good = bytearray(vtok.build_vtok([b"a", b"bc"], [1] * 256))
    vtok.TokenTable.from_vtok(bytes(good), 8)
    bad_magic = bytearray(good)
    bad_magic[0:4] = b"VTOX"
    bad_map = bytearray(good)
    o_byt = int.from_bytes(good[68:76], "little")
    bad_map[o_byt:o_byt + 4] = (2).to_bytes(4, "little")          # id >= n_vocab
    bad_str = bytearray(good)
    o_tab = int.from_bytes(good[28:36], "little")
    bad_str[o_tab + 12:o_tab + 16] = (99).to_bytes(4, "little")   # token 1 runs past the pool
    for blob in (bad_magic, bad_map, bad_str):
        with pytest.raises(vtok.VTOKError):
            vtok.TokenTable.from_vtok(bytes(blob), 8)
    with pytest.raises(vtok.VTOKError):
        vtok.TokenTable.from_vtok(bytes(good), 1)                  # more tokens than the vocabulary


def pin_cfg(**kw):
    """A tiny model whose auto-pin limit is the same under both references: the C runtime's limit is
    min(W, 512) (runtime/vault3.c:706-710, 2046), the Python model's min(max_sink, W)."""
    base = dict(window=16, max_sink=16, n_sink=4)
    base.update(kw)
    return modelgen.tiny_cfg(**base)


# (label, ids of the ChatML prefix): system prompts with and without the newline after <|im_end|>,
# a prompt without the system role, and system prompts that reach or pass the pin limit (16).
PIN_CASES = {
    "system_nl": dict(sys_len=6),
    "system_no_nl": dict(sys_len=5, nl_after_end=False),
    "no_system_role": dict(sys_len=4, system=False),
    "end_at_limit": dict(sys_len=12, nl_after_end=True),        # <|im_end|> at pos 15 = limit - 1
    "past_limit": dict(sys_len=20),
}


def pin_stream(cfg, case, n_tail=150, seed=3):
    return modelgen.chatml_prefix(cfg, **PIN_CASES[case]) + modelgen.ids_stream(cfg, n_tail, seed=seed)


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("case", list(PIN_CASES))
def test_auto_pin_and_tiers_oracle_matches_reference_runtime(case):
    cfg = pin_cfg()
    vocab = modelgen.test_vocab(cfg)
    _, image, deq = modelgen.build(cfg, "q8_0", seed=4, vocab=vocab)
    rt = ref.RefRuntime(image, threads=1)
    om = OracleModel(cfg, deq, token_bytes=vocab[0], newline_id=modelgen.NEWLINE_ID)
    st = om.new_state()
    ids = pin_stream(cfg, case)
    got, want = [], []
    for i, t in enumerate(ids):
        want.append(rt.step(t).astype(np.float64))
        got.append(om.step(t, st))
        info, fl = rt.info(), rt.flags()
        assert (info["n_pin"], fl["pin_locked"]) == (st.n_pin, st.pin_locked), (case, i)
        assert not fl["seg_bias_active"], (case, i)
    got, want = np.stack(got), np.stack(want)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-4
    assert np.array_equal(got.argmax(-1), want.argmax(-1))
    assert st.mem_pos.size > 0 and np.array_equal(rt.mem_pos(), st.mem_pos)
    if case == "past_limit":
        assert st.n_pin == 16
    elif case == "no_system_role":
        assert st.n_pin == cfg.n_sink
    else:
        assert st.n_pin > cfg.n_sink


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
def test_tiers_change_segmentation():
    """The token strings matter: the same ids with empty strings (every tier 0) leave a different
    segment memory, in the C runtime and in the oracle alike."""
    cfg = pin_cfg()
    vocab = modelgen.test_vocab(cfg)
    ids = modelgen.ids_stream(cfg, 120, seed=8)
    banks = []
    for v in (vocab, None):
        _, image, deq = modelgen.build(cfg, "q8_0", seed=4, vocab=v)
        rt = ref.RefRuntime(image, threads=1)
        om = OracleModel(cfg, deq, token_bytes=None if v is None else v[0], newline_id=modelgen.NEWLINE_ID)
        st = om.new_state()
        for t in ids:
            rt.step(t)
            om.step(t, st)
        assert np.array_equal(rt.mem_pos(), st.mem_pos)
        banks.append(st.mem_pos)
    assert not np.array_equal(banks[0], banks[1])
