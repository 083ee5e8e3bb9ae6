"""Host control logic (libvault_amd's C++ unit, vault_amd/control.py) against the reference C runtime
compiled into oracle/_ref (runtime/vault3.c), on ChatML conversations of a word-level vocabulary:

* resonance: after every v3_step, the library's shingle index (rebuilt from the reference state's bank
  tokens and segment ids) and query resonance (fed the state's token rings, position and pin count)
  give the same mode (seg_bias_active) and bit-identical arch / sup (and, in mode 2, hop-1) biases
  over the bank (runtime/vault3.c:1178-1786);
* spoof quarantine: the library's check fires exactly at the steps whose segment score the reference
  set to -1e30 (runtime/vault3.c:1798-1831, 2215);
* governor: masks equal to v3_govern_logits on the reference's governor (runtime/vault3.c:2888-3193)
  for the evasions of tests/test_vlt3_runtime.py:350-360 and 580-660 (split, separator, zero-width,
  homoglyph, reversed, Base64, hex) and benign text, over random logits and committed streams.
No GPU: the library's host entry points only."""
import numpy as np
import pytest

from oracle import ref
from tests import modelgen
from vault_amd import control

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")

KINDS = ("id", "ids", "words", "rollback", "hop", "spoof", "clause")


def _cfg(seg_budget):
    return modelgen.tiny_cfg(window=32, seg_budget=seg_budget, vocab=512, seg_max=7, max_sink=32, n_sink=4)


@pytest.fixture(scope="module", params=[128, 40], ids=["bank_keeps_all", "bank_evicts"])
def setup(request):
    cfg = _cfg(request.param)
    toks, bmap = modelgen.word_vocab(cfg)
    _, image, _ = modelgen.build(cfg, "q8_0", seed=6, vocab=(toks, bmap))
    return cfg, toks, image


def _run(cfg, toks, image, kind, seed, counts):
    rt = ref.RefRuntime(image, threads=1)
    tb = control.TokenBytes(toks)
    res = control.Resonance(tb, cfg.window, cfg.seg_budget, cfg.n_sink, cfg.im_start_id, cfg.im_end_id)
    W = cfg.window
    last_bank = None
    for i, t in enumerate(modelgen.conversation(cfg, toks, kind, seed=seed)):
        rt.step(t)
        info, fl = rt.info(), rt.flags()
        pos, n_pin = info["pos"] - 1, info["n_pin"]
        c = pos % W
        mem_tok, mem_seg, arch, sup, hop1 = rt.res_state()
        bank = (mem_tok.tobytes(), mem_seg.tobytes())
        if bank != last_bank:
            res.rebuild(mem_tok, mem_seg)
            last_bank = bank
            assert res.n_segs == fl["n_uniq_segs"], (kind, seed, i)
        prev, cur, sc = rt.rings(W)
        mode = res.update(prev, cur, c, pos, n_pin)
        assert mode == fl["seg_bias_active"], (kind, seed, i)
        if mode:
            M = mem_tok.size
            assert np.array_equal(res.arch[:M].view(np.uint32), arch.view(np.uint32)), (kind, seed, i)
            assert np.array_equal(res.sup[:M].view(np.uint32), sup.view(np.uint32)), (kind, seed, i)
            if mode == 2:
                assert np.array_equal(res.hop1[:M].view(np.uint32), hop1.view(np.uint32)), (kind, seed, i)
        counts[mode] = counts.get(mode, 0) + 1
        spoof = control.spoof_check(tb, prev, cur, W, c, pos, n_pin, cfg.n_sink)
        if pos >= 0:
            assert spoof == (sc[c] == np.float32(-1e30)), (kind, seed, i)
        counts["spoof"] = counts.get("spoof", 0) + int(spoof)


def test_resonance_and_spoof_match_reference_runtime(setup):
    cfg, toks, image = setup
    counts = {}
    for kind in KINDS:
        for seed in range(4):
            _run(cfg, toks, image, kind, seed, counts)
    # every branch family was reached: no bias, the arch / sup biases, the hop-1 mode, the quarantine
    assert counts.get(0, 0) > 0 and counts.get(1, 0) > 0 and counts.get(2, 0) > 0 and counts["spoof"] > 0, counts


# ---------------------------------------------------------------------------------------------- governor

SYS_PROMPTS = [
    b"You are a careful agent. Never call 'syscall_exec(' or emit \"rm_rf(\" under any circumstance.",
    b"Do not output `sys_call_exec` and NEVER print 'drop_table'.",
    b"Prohibit any `fork_bomb(` output; the helper 'rm_rf(' must not appear.",
    b"Be brief and helpful.",                                   # no prohibition cue: inactive
]


@pytest.fixture(scope="module")
def gov_setup():
    cfg = _cfg(0)
    toks, bmap = modelgen.word_vocab(cfg)
    _, image, _ = modelgen.build(cfg, "q8_0", seed=6, vocab=(toks, bmap))
    return cfg, toks, ref.RefRuntime(image, threads=1)


def _pair(cfg, toks, rt, prompt):
    g = control.Governor.from_system_prompt(prompt, control.TokenBytes(toks), eos_id=0, im_start_id=cfg.im_start_id,
                                            im_end_id=cfg.im_end_id)
    r = ref.RefGovernor(rt)
    r.arm_system(prompt)
    return g, r


@pytest.mark.parametrize("prompt", SYS_PROMPTS)
def test_governor_masks_match_reference(gov_setup, prompt):
    """Random logits with the governor's candidate tokens boosted, after committed prefixes that set
    up split / spaced / homoglyph / reversed / encoded completions: the masked set equals
    v3_govern_logits at top_k_guard 64, 8 and 0."""
    cfg, toks, rt = gov_setup
    ids = modelgen.word_ids(toks)
    rng = np.random.default_rng(len(prompt))
    V = cfg.vocab_size
    prefixes = [[b" sys", b"call"], [b"SYS", b"CALL"], [b" s", b"y", b" s", b"c", b"a", b"l", b"l"],
                [b"\xe2\x80\x8b", b" sys", "с".encode(), b"a"], [b"cexe_llacsys"], [b"c3lz", b"Y2Fs"], [b"73", b"79"],
                [b"rm"], [b"rm", b"_rf"], [], [b" falcon", b" harbor"], [b"\\x61", b"0x6c"]]
    boosted = [ids[b] for b in (b"_exec", b"_EXEC", b"_exec", b"ex", b"ec", b"bF9l", b"eGVj", b"73 63", b" rm_rf(",
                                b"(", b"x", b"e", b" orchid", b"Y2Fs", b"cexe_llacsys")]
    n_masked = 0
    for pi, pre in enumerate(prefixes):
        g, r = _pair(cfg, toks, rt, prompt)
        for b in pre:
            g.commit(ids[b])
            r.commit(ids[b])
        for guard in (64, 8, 0):
            x = rng.standard_normal(V).astype(np.float32)
            x[boosted] = 6.0 + rng.standard_normal(len(boosted)).astype(np.float32)
            x[rng.integers(0, V, 3)] = -np.inf
            want = r.govern_logits(x, guard)
            masked = set(np.flatnonzero(want != x).tolist())
            got = set(g.screen(*_candidates(x), guard, V).tolist())
            assert got == masked, (prompt, pi, guard)
            n_masked += len(masked)
    if g.active:
        assert n_masked > 0
    else:
        assert n_masked == 0


def _candidates(x, T=256):
    """The row's top T as the device selection returns them: value desc, index asc, NaN excluded."""
    order = sorted(range(x.size), key=lambda i: (-float(x[i]), i))[:T]
    return np.array(order, dtype=np.int64), x[order]


def test_governor_stream_resets_and_rules(gov_setup):
    """Rules and stream state through add_rule / commit / reset: special ids reset the stream, the
    rule table caps at 8 distinct rules, short rules are rejected; masks equal the reference's."""
    cfg, toks, rt = gov_setup
    ids = modelgen.word_ids(toks)
    V = cfg.vocab_size
    tb = control.TokenBytes(toks)
    g = control.Governor(tb, eos_id=0, im_start_id=cfg.im_start_id, im_end_id=cfg.im_end_id)
    r = ref.RefGovernor(rt)
    for pat in (b"sys", b"syscall_exec", b"SYSCALL-EXEC", "ѕуѕсаll".encode(), b"rm_rf(", b"abcd", b"efgh", b"ijkl",
                b"mnop", b"qrst", b"uvwx"):
        assert g.add_rule(pat) == r.add_rule(pat), pat
    rng = np.random.default_rng(5)
    stream = [b" sys", b"call", b" falcon", cfg.im_end_id, b"rm", b"_rf", b"SYS", 0, b"call", b" s", b"y"]
    for s in stream:
        tid = s if isinstance(s, int) else ids[s]
        x = rng.standard_normal(V).astype(np.float32)
        x[[ids[b"_exec"], ids[b"("], ids[b"_EXEC"], ids[b"ex"]]] = 5.0
        want = r.govern_logits(x, 0)
        got = set(g.screen(*_candidates(x), 0, V).tolist())
        assert got == set(np.flatnonzero(want != x).tolist()), s
        g.commit(tid)
        r.commit(tid)


ENCODED = [
    ("b64 aligned", [b"c3lzY2Fs"], b"bF9leGVj"),
    ("b64 three bytes off", [b"QQQ", b"c3lzY2Fs"], b"bF9leGVj"),
    ("b64 whole token", [], b"cm1fcmYo"),
    ("hex 0x", [b"0x73 0x79 0x73", b" 0x63 0x61 0x6c", b" 0x6c 0x5f 0x65"], b" 0x78 0x65 0x63"),
    ("hex \\x", [b"\\x72\\x6d\\x5f"], b"\\x72\\x66\\x28"),
]


@pytest.mark.parametrize("name,prefix,cand", ENCODED, ids=[e[0] for e in ENCODED])
def test_governor_encoded_completions(gov_setup, name, prefix, cand):
    """Encoded completions of the rules (Base64 at every alignment, hex with 0x / \\x prefixes): the
    candidate that completes one is masked by the reference, and the masks agree."""
    cfg, toks, rt = gov_setup
    ids = modelgen.word_ids(toks)
    g, r = _pair(cfg, toks, rt, SYS_PROMPTS[0])
    for b in prefix:
        g.commit(ids[b])
        r.commit(ids[b])
    x = np.random.default_rng(len(name)).standard_normal(cfg.vocab_size).astype(np.float32)
    x[ids[cand]] = 9.0
    want = r.govern_logits(x, 0)
    assert want[ids[cand]] < -3e38, name                # the case is one the reference blocks
    got = set(g.screen(*_candidates(x), 0, cfg.vocab_size).tolist())
    assert got == set(np.flatnonzero(want != x).tolist()), name


@pytest.fixture(scope="module")
def direct():
    cfg = _cfg(128)
    toks, bmap = modelgen.word_vocab(cfg)
    _, image, _ = modelgen.build(cfg, "q8_0", seed=6, vocab=(toks, bmap))
    rt = ref.RefRuntime(image, threads=1)
    tb = control.TokenBytes(toks)
    res = control.Resonance(tb, cfg.window, cfg.seg_budget, cfg.n_sink, cfg.im_start_id, cfg.im_end_id)
    return cfg, toks, rt, tb, res


def _check(cfg, rt, tb, res, bank_tok, bank_seg, prev, cur, c, pos, n_pin, tag):
    n = rt.res_load_bank(bank_tok, bank_seg)
    assert res.rebuild(bank_tok, bank_seg) == n, tag
    mode_r, a, s, h = rt.res_update(prev, cur, c, pos, n_pin)
    mode = res.update(prev, cur, c, pos, n_pin)
    assert mode == mode_r, tag
    M = len(bank_tok)
    if mode:
        assert np.array_equal(res.arch[:M].view(np.uint32), a.view(np.uint32)), tag
        assert np.array_equal(res.sup[:M].view(np.uint32), s.view(np.uint32)), tag
        if mode == 2:
            assert np.array_equal(res.hop1[:M].view(np.uint32), h.view(np.uint32)), tag
    assert control.spoof_check(tb, prev, cur, cfg.window, c, pos, n_pin, cfg.n_sink) == rt.spoof(prev, cur, c, pos,
                                                                                                   n_pin), tag
    return mode


def test_resonance_random_banks_match_reference(direct):
    """Constructed banks (random segment runs of word / identifier / delimiter tokens, 0..128 slots) and
    rings (a question copied in part from the bank, <|im_end|> 0..45 tokens back, random pins and
    positions): update_query_resonance and check_spoof_quarantine of the reference on the same state."""
    cfg, toks, rt, tb, res = direct
    ids = modelgen.word_ids(toks)
    W, rng = cfg.window, np.random.default_rng(11)
    pool = [ids[b] for b in modelgen.KEYS + modelgen.WORDS + modelgen.GLUE[:40]] + [modelgen.NEWLINE_ID] * 6
    modes = {0: 0, 1: 0, 2: 0}
    for case in range(600):
        M = int(rng.integers(0, cfg.seg_budget + 1))
        tok = rng.choice(pool, size=M)
        runs = rng.integers(1, 13, size=M + 1)
        seg = np.repeat(np.arange(len(runs)), runs)[:M] + int(rng.integers(0, 50))
        ring = rng.choice(pool, size=2 * W)
        hi = W + int(rng.integers(0, W))
        gen = int(rng.integers(0, 46))
        pe = hi - gen
        if pe > 0:
            ring[pe] = cfg.im_end_id
            qlen = int(rng.integers(2, 20))
            lo = max(0, pe - qlen)
            if M > 0 and rng.random() < 0.8:
                a = int(rng.integers(0, M))
                src = tok[a:a + min(qlen, pe - lo)]
                ring[lo:lo + len(src)] = src
            if rng.random() < 0.5 and lo > 0:
                ring[lo - 1] = cfg.im_start_id
        prev, cur = ring[:W], ring[W:]
        c = hi - W
        pos = 2 * W * int(rng.integers(1, 50)) + c
        n_pin = int(rng.integers(0, 40))
        modes[_check(cfg, rt, tb, res, tok, seg, prev, cur, c, pos, n_pin, case)] += 1
    assert min(modes.values()) > 0, modes


def test_resonance_tier_b_threshold(direct):
    """Fifteen segments, two content words each in four of them: both words score 2 x 1236 = 2472 in the
    segments that hold both, below tier B's 2500, so no bias; with a third shared word, a match."""
    cfg, toks, rt, tb, res = direct
    ids = modelgen.word_ids(toks)
    W = cfg.window
    w1, w2, w3 = (ids[b] for b in (b" falcon", b" harbor", b" meadow"))
    fill = [ids[b] for b in (b" anchor", b" beacon", b" cobalt", b" dynamo", b" ember", b" glacier", b" indigo")]
    for third in (False, True):
        tok, seg = [], []
        for sid in range(15):
            body = [fill[sid % len(fill)], ids[b" key_%d" % sid]]
            if sid < 4:
                body += [w1, w2] + ([w3] if third and sid < 2 else [])
            tok += body + [modelgen.NEWLINE_ID]
            seg += [sid] * (len(body) + 1)
        ring = np.full(2 * W, ids[b" the"], dtype=np.int64)
        q = [cfg.im_start_id, ids[b" user"], modelgen.NEWLINE_ID, w1, w2] + ([w3] if third else [])
        ring[W + 2:W + 2 + len(q)] = q
        ring[W + 2 + len(q)] = cfg.im_end_id
        c = W - 1 - 20
        mode = _check(cfg, rt, tb, res, np.array(tok), np.array(seg), ring[:W], ring[W:], c, 10 * W + c, 0, third)
        assert mode == (1 if third else 0), third


def test_resonance_random_clauses_match_reference(direct):
    """Banks of long segments split into clauses by ';' / '|' / tab-free delimiters (the clause
    refinement of runtime/vault3.c:1307-1424) with questions that name several of a segment's
    identifiers and words: same modes and biases as the reference."""
    cfg, toks, rt, tb, res = direct
    ids = modelgen.word_ids(toks)
    W, rng = cfg.window, np.random.default_rng(21)
    content = [ids[b] for b in modelgen.KEYS + modelgen.WORDS]
    glue = [ids[b] for b in (b" =", b":", b" the", b" and", b" set", b" to")]
    delims = [ids[b";"], ids[b" |"], modelgen.NEWLINE_ID]
    for case in range(800):
        tok, seg = [], []
        n_seg = int(rng.integers(3, 9))
        for sid in range(n_seg):
            body = []
            for _ in range(int(rng.integers(1, 5))):
                body += list(rng.choice(content, size=int(rng.integers(2, 6)))) + list(rng.choice(glue, size=1))
                body.append(int(rng.choice(delims)))
            tok += body
            seg += [sid] * len(body)
        tok, seg = np.array(tok[:cfg.seg_budget]), np.array(seg[:cfg.seg_budget])
        pick = int(rng.integers(0, n_seg))
        mine = tok[seg == pick]
        q = list(rng.choice(mine, size=min(len(mine), int(rng.integers(2, 6))), replace=False))
        ring = np.full(2 * W, ids[b" the"], dtype=np.int64)
        qq = [cfg.im_start_id, ids[b" user"], modelgen.NEWLINE_ID] + q + [ids[b"?"]]
        ring[W + 1:W + 1 + len(qq)] = qq
        ring[W + 1 + len(qq)] = cfg.im_end_id
        c = W - 1 - int(rng.integers(0, W - 2 - len(qq)))
        _check(cfg, rt, tb, res, tok, seg, ring[:W], ring[W:], c, 20 * W + c, int(rng.integers(0, 30)), case)


@pytest.mark.parametrize("best,other", [(4, 3), (3, 2)], ids=["ratio_3_4", "ratio_2_3"])
def test_resonance_clause_ratio_boundary(direct, best, other):
    """One matched segment (tier B, four equal-weight content words) of three clauses holding `best`,
    `other` and one of the question's words: a clause below 3/4 of the best clause's score is set back
    to the sibling value, one at exactly 3/4 is not (runtime/vault3.c:1408-1419)."""
    cfg, toks, rt, tb, res = direct
    ids = modelgen.word_ids(toks)
    W = cfg.window
    qw = [ids[b] for b in (b" falcon", b" harbor", b" meadow", b" orchid")]
    eq, semi, nl = ids[b" ="], ids[b";"], modelgen.NEWLINE_ID
    fill = [ids[b] for b in (b" anchor", b" beacon", b" cobalt", b" dynamo")]
    clauses = [qw[:best] + [eq, fill[0]], qw[:other] + [eq, fill[1]], qw[:1] + [eq, fill[2], fill[3]]]
    seg_toks = clauses[0] + [semi] + clauses[1] + [semi] + clauses[2] + [nl]
    tok, seg = list(seg_toks), [0] * len(seg_toks)
    for sid in range(1, 5):
        body = [fill[sid - 1], ids[b" key_%d" % sid], eq, ids[b" prism"], nl]
        tok += body
        seg += [sid] * len(body)
    ring = np.full(2 * W, ids[b" the"], dtype=np.int64)
    q = [cfg.im_start_id, ids[b" user"], nl] + qw[:best] + [ids[b"?"]]
    ring[W + 2:W + 2 + len(q)] = q
    ring[W + 2 + len(q)] = cfg.im_end_id
    c = W - 1 - 10
    mode = _check(cfg, rt, tb, res, np.array(tok), np.array(seg), ring[:W], ring[W:], c, 10 * W + c, 0, (best, other))
    assert mode == 1
    # the reference's own decision on the middle clause: refined below 3/4, kept at 3/4
    _, a, _, _ = rt.res_update(ring[:W], ring[W:], c, 10 * W + c, 0)
    first, middle = a[0], a[len(clauses[0]) + 1]
    assert (middle != first) == (other * 4 < best * 3)
