"""Host control rules in the GPU model, against the reference C runtime (runtime/vault3.c, compiled into
oracle/_ref) on ChatML conversations of a word-level vocabulary: the resonance bias on the segment span
(modes 1 and 2), the spoof quarantine of the segment score, through the step stream and through
prefill / forward (chunks with active resonance take the step path); the device top-T candidate
selection (vgx_topk) against a host sort; the output governor on device logits against
v3_govern_logits.

Bars: logits rel < 1e-4 and 100% top-1 (tests/test_vlt3_runtime.py:90-94); resonance modes, pin
counts and segment-memory positions exactly; candidate lists and masks exactly."""
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import ref
from tests import modelgen
from vault_amd import control, ops
from vault_amd.model import VAULTv3ForCausalLM
from vault_amd.weights import ModelWeights

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("B,V", [(3, 151665), (2, 4096), (1, 1000), (2, 70000)])
def test_topk_matches_host_sort(dev, B, V):
    rng = np.random.default_rng(V + B)
    x = rng.standard_normal((B, V)).astype(np.float32)
    x[0, rng.integers(0, V, 50)] = 3.5                  # ties across chunks
    x[0, 7] = np.nan
    x[-1, rng.integers(0, V, 20)] = -np.inf
    x[-1, 0] = -0.0
    if V > 300:
        x[-1, 1:300] = 0.0                              # a tie run with -0 first
    idx, val = ops.topk(torch.from_numpy(x).to(dev), 256)
    idx, val = idx.cpu().numpy(), val.cpu().numpy()
    for b in range(B):
        ok = [i for i in range(V) if not np.isnan(x[b, i])]
        want = sorted(ok, key=lambda i: (-(float(x[b, i]) + 0.0), i))[:256]
        want += [-1] * (256 - len(want))
        assert np.array_equal(idx[b], np.array(want)), b
        n = min(256, len(ok))
        assert np.array_equal(val[b, :n], x[b, want[:n]]), b


@pytest.fixture(scope="module", params=[(128, 64), (40, 64), (40, 128)],
                ids=["bank_keeps_all", "bank_evicts", "bank_evicts_d128"])
def word_model(request, dev):
    budget, head_dim = request.param
    heads = dict(n_heads=12, n_kv_heads=2) if head_dim == 128 else {}
    cfg = modelgen.tiny_cfg(window=32, seg_budget=budget, vocab=512, seg_max=7, max_sink=32, n_sink=4,
                            head_dim=head_dim, n_layers=4, **heads)
    toks, bmap = modelgen.word_vocab(cfg)
    _, image, _ = modelgen.build(cfg, "q8_0", seed=6, vocab=(toks, bmap))
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.vlt3")
        with open(path, "wb") as f:
            f.write(image)
        w = ModelWeights.from_vlt3(path, dev)
    return cfg, toks, image, VAULTv3ForCausalLM(w)


@needs_ref
@pytest.mark.parametrize("kind", ["ids", "rollback", "hop", "spoof", "clause", "words"])
def test_resonance_stream_matches_reference_runtime(word_model, kind):
    cfg, toks, image, m = word_model
    rt = ref.RefRuntime(image, threads=2)
    st = m.new_state(1)
    assert st.res is not None
    modes, n_quar = [], 0
    got, want = [], []
    for i, t in enumerate(modelgen.conversation(cfg, toks, kind, seed=1)):
        c = i % cfg.window
        want.append(rt.step(t).astype(np.float64))
        got.append(m.step(torch.tensor([t]), st)[0].double().cpu().numpy())
        fl = rt.flags()
        assert st.seg_bias_mode == fl["seg_bias_active"], (kind, i)
        assert st.n_pin == rt.info()["n_pin"], (kind, i)
        modes.append(st.seg_bias_mode)
        if st.seg_bias_mode:
            # the reference's per-head layout (free heads 0, arch, sup; hop-1 on the biased heads in mode 2)
            _, _, arch, sup, hop1 = rt.res_state()
            cls = control.head_classes(cfg.n_heads, cfg.n_kv_heads)
            late = st.seg_head_bias[0, :, 0].cpu().numpy()
            for h, k in enumerate(cls):
                want_h = np.zeros_like(arch) if k == 0 else arch if k == 1 else sup
                assert np.array_equal(late[h].view(np.uint32), want_h.view(np.uint32)), (kind, i, h)
            if st.seg_bias_mode == 2:
                early = st.seg_head_bias_hop1[0, :, 0].cpu().numpy()
                for h, k in enumerate(cls):
                    assert np.array_equal(early[h], np.zeros_like(hop1) if k == 0 else hop1), (kind, i, h)
            else:
                assert st.seg_head_bias_hop1 is None
        # this step's segment score: quarantined exactly when the reference's is, else to fp32 precision
        s_ref, s_dev = float(rt.rings(cfg.window)[2][c]), float(st.sc_cur[c])
        assert (s_ref <= -1e29) == (s_dev <= -1e29), (kind, i)
        n_quar += s_ref <= -1e29
        if s_ref > -1e29:
            assert abs(s_dev - s_ref) <= 1e-4 * max(1.0, abs(s_ref)), (kind, i)
    got, want = np.stack(got), np.stack(want)
    assert _rel(got, want) < 1e-4, kind
    assert np.array_equal(got.argmax(-1), want.argmax(-1)), kind
    assert np.array_equal(rt.mem_pos(), st.mem_pos.numpy()), kind
    if kind in ("ids", "hop", "rollback"):
        assert max(modes) > 0, kind
    if kind == "spoof":
        assert n_quar > 0


@needs_ref
@pytest.mark.parametrize("kind,split", [("ids", 150), ("rollback", 100), ("spoof", 160), ("hop", 140)])
def test_resonance_prefill_matches_stream(word_model, kind, split):
    """prefill(split tokens) then the stream, and forward() over the whole conversation: every logit row
    against the reference runtime stepping the same ids.  At head_dim 128 (the MFMA chunk attention)
    chunks in which resonance is active keep the chunk path with per-row bias (the prefill's chunks are
    checked to have carried one); at head_dim 64 they run the step path."""
    cfg, toks, image, m = word_model
    ids = modelgen.conversation(cfg, toks, kind, seed=1)
    rt = ref.RefRuntime(image, threads=2)
    want, ref_modes = [], []
    for t in ids:
        want.append(rt.step(t).astype(np.float64))
        ref_modes.append(rt.flags()["seg_bias_active"])
    want = np.stack(want)
    biased = []
    chunk_bias = m._chunk_bias

    def spy(*a, **k):
        r = chunk_bias(*a, **k)
        biased.append(r is not None)
        return r

    m._chunk_bias = spy
    try:
        last, st = m.prefill(torch.tensor([ids[:split]]))
    finally:
        del m._chunk_bias
    if m._mfma_prefill():
        # the chunk-bias path ran exactly when the reference's resonance was active inside the prefill
        assert any(biased) == any(ref_modes[:split]), (biased, max(ref_modes[:split]))
    rows = [last[0].double().cpu().numpy()]
    for t in ids[split:]:
        rows.append(m.step(torch.tensor([t]), st)[0].double().cpu().numpy())
    got = np.stack(rows)
    assert _rel(got, want[split - 1:]) < 1e-4
    assert np.array_equal(got.argmax(-1), want[split - 1:].argmax(-1))
    assert np.array_equal(rt.mem_pos(), st.mem_pos.numpy())
    full = m.forward(torch.tensor([ids]))[0].double().cpu().numpy()
    assert _rel(full, want) < 1e-4
    assert np.array_equal(full.argmax(-1), want.argmax(-1))


@needs_ref
def test_governor_on_device_logits(word_model, dev):
    """Governor.govern_logits (device top-256 candidates, host rule screen, device mask) equals
    v3_govern_logits on the same rows after the same committed tokens."""
    cfg, toks, image, m = word_model
    rt = ref.RefRuntime(image, threads=1)
    ids = modelgen.word_ids(toks)
    prompt = b"Never call 'syscall_exec(' and never emit \"rm_rf(\"."
    g = control.Governor.from_system_prompt(prompt, m.ctl_tokens, eos_id=0, im_start_id=cfg.im_start_id,
                                            im_end_id=cfg.im_end_id)
    r = ref.RefGovernor(rt)
    r.arm_system(prompt)
    assert g.active
    rng = np.random.default_rng(3)
    stream = [b"c3lzY2Fs", b" sys", b"call", b"SYS", b"CALL", b" falcon", b"rm", b"QQQ", b"c3lzY2Fs"]
    n_masked = 0
    for s in stream:
        x = rng.standard_normal(cfg.vocab_size).astype(np.float32)
        x[[ids[b"_exec"], ids[b"_EXEC"], ids[b"bF9leGVj"], ids[b"_rf"], ids[b"ex"]]] = 7.0
        want = r.govern_logits(x, 0)
        row = torch.from_numpy(x).to(dev)
        masked = g.govern_logits(row, 0)
        assert set(masked.tolist()) == set(np.flatnonzero(want != x).tolist()), s
        assert np.array_equal(row.cpu().numpy(), want), s
        n_masked += masked.size
        g.commit(ids[s])
        r.commit(ids[s])
    assert n_masked > 0
