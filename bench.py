"""Decode throughput of the VAULT v3 hot path on one MI355X.

Workload (one "step"): one full 28-layer decode step of a random-init 1.54B VAULT v3 model
(d=1536, 12 query / 2 KV heads, head_dim 128, SwiGLU 8960, vocab 151665) in hybrid Q4_0
(Q8_0 embeddings / tied LM head, Q8_0 k/v projections, Q8_0 q/o projections in layers 0, 1, 26, 27;
Q4_0 elsewhere) at 100K-token context: 512 pinned sinks, 1024 segment-memory slots and the 2W=2048
window (W=1024), segment scorer on, batch 1 (``--batch`` for more; segment memory is off for
batch > 1 as in the reference).  The state is seeded where a long stream leaves it (fixed-size
state), weights are drawn directly as quantized blocks from a seeded generator.

The timed steps cross a chunk boundary (segment-memory merge, bank compaction, ring swap and
re-rotations inside the timed region); both ring configurations' step graphs are captured during
set-up.

Prints one JSON line: tokens/s, plus the roofline of the step's largest kernel by time (batch-1 decode
attention over the step's four KV spans, fp32 KV, with its split merge), secondary kernel figures
(the fused gate/up SwiGLU Q4_0 GEMV, Q8_0/Q4_0 GEMV at the model's shapes, batched bf16 decode
attention at 3584 keys, prefill attention and GEMMs, batch-32 decode, and the same model with token
strings: a 16K-token multi-turn ChatML prefill and decode with the resonance rules active) and the
reference C runtime timed on the host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
CTX_POS = 100_000          # first decoded position: 100K tokens of context already streamed
N_PIN, MEM_CNT = 512, 1024


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_config(vocab: int = 151665):
    from vault_amd.config import QWEN25_1P5B
    from dataclasses import replace
    return replace(QWEN25_1P5B, vocab_size=vocab, auto_pin_system=False)


def build_model(cfg, dev, kv_dtype, seed: int = 1234):
    from vault_amd.model import VAULTv3ForCausalLM
    from vault_amd.weights import ModelWeights, synthetic_tensors
    t0 = time.time()
    tensors = synthetic_tensors(cfg, "q4_0", seed)
    _log(f"synthetic weights generated in {time.time() - t0:.1f}s")
    w = ModelWeights.from_tensors(cfg, tensors, dev)
    return VAULTv3ForCausalLM(w, kv_dtype=kv_dtype), tensors


def seeded_state(model, batch: int, seed: int = 99, pos: int = CTX_POS, st=None):
    import torch
    if st is None:
        st = model.new_state(batch, seg_budget=None if batch == 1 else 0)
    gen = torch.Generator().manual_seed(seed)
    st.seed_long_context(pos, N_PIN, MEM_CNT if batch == 1 else 0,
                         lambda li, name, shape: torch.randn(shape, generator=gen))
    return st


def boundary_seeded_state(model, batch: int, steps: int, warmup: int):
    """A seeded state whose timed steps cross a chunk boundary (the segment-memory merge, the bank
    compaction, the ring swap and re-rotations run inside the timed region), with both ring
    configurations' step graphs already captured.  Set-up: seed two positions before the chunk
    boundary at 99,328 and step across it (the first step's graph and the graph after the swap are
    captured there), then seed the same buffers again so that boundary 100,352 falls in the middle of
    the timed steps.  Returns (state, first decoded position)."""
    import torch
    W = model.cfg.window
    b2 = (CTX_POS // W + 1) * W                   # 100,352
    st = seeded_state(model, batch, pos=b2 - W - 2)
    g = torch.Generator().manual_seed(77)
    for t in torch.randint(0, model.cfg.vocab_size, (4, batch), generator=g):
        model.step(t, st)
    torch.cuda.synchronize()
    p0 = max(2 * W, b2 - warmup - steps // 2)
    seeded_state(model, batch, pos=p0, st=st)
    return st, p0


def _events():
    import torch
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def graph_time_us(fn, launches_per_call: int, reps: int = 20) -> float:
    """Average GPU time per launch of ``fn`` (a sequence of library calls), measured by capturing one
    call into a HIP graph and replaying it ``reps`` times between HIP events on the replay stream."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                  # warm (allocations, workspaces) outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = _events()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * launches_per_call)


def time_decode(model, st, steps: int, warmup: int, batch: int, seed: int = 5):
    import torch
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, model.cfg.vocab_size, (warmup + steps, batch), generator=g)
    for i in range(warmup):
        model.step(ids[i], st)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        logits = model.step(ids[warmup + i], st)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    assert torch.isfinite(logits).all()
    return dt


ATTN_LENS = (512, 1024, 1024, 1024)        # sinks | segment memory | previous window | current window
ATTN_COPIES = 40                           # 40 x 7.34 MB of KV: beyond the 256 MB last-level cache
ATTN_ALGO_BYTES = sum(ATTN_LENS) * 2 * 128 * 4 * 2 + 2 * 12 * 128 * 4   # K and V once, q and out


def attention_kernel(dev, reps: int = 20):
    """The roofline kernel: batch-1 decode attention of the step, fp32 KV (the state dtype), 12 query /
    2 KV heads, D = 128, 3584 keys in the step's four spans (512 sinks | 1024 segment slots | 1024
    previous | 1024 current window).  One call = attn_decode_b1_kernel over 56 key splits of 64 keys x
    2 KV groups (112 workgroups of 8 waves) + b1_merge_kernel (12 heads x 4 dim quarters).  Algorithmic
    bytes per call: K and V once (7,340,032 B) + q + out = 7,352,320 B.
    A graph replays one call over each of ATTN_COPIES KV copies (as the 28 layers of a step stream
    theirs); time per call from HIP events on the replay stream."""
    import torch
    from vault_amd import ops
    B, H, G, D = 1, 12, 2, 128
    g = torch.Generator().manual_seed(12)
    base = [(torch.randn(B, G, n, D, generator=g).to(dev), torch.randn(B, G, n, D, generator=g).to(dev))
            for n in ATTN_LENS]
    sets = _kv_copies(base, ATTN_COPIES)
    q = torch.randn(B, H, D, generator=g).to(dev)
    out = torch.empty(B, H, D, device=dev)
    ws = ops.Workspace(dev)

    def run():
        for sp in sets:
            ops.attn_decode(q, sp, out=out, ws=ws)
    us = graph_time_us(run, len(sets), reps=reps)
    # the same calls over one KV copy (7.3 MB, resident in the last-level cache): reported separately
    warm = graph_time_us(lambda: [ops.attn_decode(q, base, out=out, ws=ws) for _ in sets], len(sets), reps=reps)
    return {"kernel": "attn_decode_b1_kernel<fp32 KV, 6 heads per KV group, 8 waves, 2 key blocks per wave, "
                      "spans of whole key blocks> + b1_merge_kernel (batch 1, 12 q / 2 KV heads, D = 128, 3584 keys)",
            "calls": reps * len(sets), "avg_us": us, "bytes_per_launch": ATTN_ALGO_BYTES,
            "gbs": ATTN_ALGO_BYTES / us / 1e3, "cache_resident_us": round(warm, 3)}


def copy_peak(dev, reps: int = 20):
    """Measured HBM copy rate: torch's elementwise negation over 1 GiB (read + written once), HIP events
    around ``reps`` launches on the current stream; bytes moved / time."""
    import torch
    n = (1 << 30) // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    e0, e1 = _events()
    e0.record()
    for _ in range(reps):
        torch.neg(src, out=dst)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    del src, dst
    return {"bytes": 2 * n * 4, "us": round(us, 1), "gbs": round(2 * n * 4 / us / 1e3, 1)}


def gateup_kernel(model, rounds: int = 20):
    """Fused gate/up SwiGLU Q4_0 GEMV (2 x 8960 x 1536) over the 28 layers' weights in turn, as in the
    step (433 MB of weights, beyond the 256 MB last-level cache); HIP events on the launch stream."""
    import torch
    from vault_amd import ops
    cfg = model.cfg
    x = torch.randn(1, cfg.d_model, device=model.device)
    h = torch.empty(1, cfg.d_ff, device=model.device)
    layers = model.w.layers
    lnw = layers[0].ln2

    def one_round():
        for lw in layers:
            ops.qlinear_swiglu(lw.wgu, x, out=h, norm=(lnw, cfg.rms_eps))

    us = graph_time_us(one_round, len(layers), reps=rounds)
    n = rounds * len(layers)
    wb = layers[0].wgu.stream_bytes
    algo = wb + 4 * cfg.d_model + 4 * cfg.d_ff
    return {"kernel": "gemv1_stream_kernel<Q4_0, SwiGLU epilogue, RMSNorm prologue> (persistent, 1 KB per load "
                      "instruction; gate|up 2x8960x1536)",
            "launches": n, "avg_us": us, "bytes_per_launch": algo, "gbs": algo / us / 1e3}


def gemv_figures(dev, batches=(1, 16), reps: int = 20, shapes=None):
    """Q8_0 / Q4_0 GEMV at the model's projection shapes, weights rotated over copies that exceed the
    last-level cache; GB/s of algorithmic bytes (weights + x + y)."""
    import numpy as np
    import torch
    from vault_amd import ops, vlt3
    shapes = shapes or [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960), (151665, 1536)]
    rng = np.random.default_rng(7)
    out = []
    for dt, name in ((vlt3.Q8_0, "q8_0"), (vlt3.Q4_0, "q4_0")):
        for rows, cols in shapes:
            raw = vlt3.synthetic_blocks(dt, rows, cols, rng)
            w0 = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
            ncopy = max(2, math.ceil(768e6 / w0.stream_bytes))
            ws = [w0] + [ops.QWeight(dt, rows, cols, w0.packed.clone()) for _ in range(ncopy - 1)]
            for b in batches:
                x = torch.randn(b, cols, device=dev)
                y = torch.empty(b, rows, device=dev)

                def run():
                    for w in ws:
                        ops.qlinear(w, x, out=y)

                us = graph_time_us(run, len(ws), reps=reps)
                algo = w0.stream_bytes + 4 * b * (rows + cols)
                out.append({"dtype": name, "out": rows, "in": cols, "batch": b, "us": round(us, 2),
                            "gbs": round(algo / us / 1e3, 1), "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 3)})
            del ws, w0
    return out


def gemm_figures(dev, rows_in: int = 1024, reps: int = 10):
    """Q4_0 projection GEMMs of one 1024-token prefill chunk (q|k|v, o, gate/up with SwiGLU, down),
    bf16 MFMA: TFLOP/s of 2 * tokens * in * out (gate/up: both halves) against 2.5 PFLOP/s dense bf16.
    Each figure includes the activation split pre-pass and, where K is split, the reduce launch."""
    import numpy as np
    import torch
    from vault_amd import ops, vlt3
    rng = np.random.default_rng(9)
    dt = vlt3.Q4_0
    out = []
    for name, rows, cols, gu in (("qkv", 2048, 1536, False), ("o", 1536, 1536, False),
                                 ("gate_up", 8960, 1536, True), ("down", 1536, 8960, False)):
        if gu:
            w = ops.QWeight.gateup_from_blocks(dt, rows, cols, vlt3.synthetic_blocks(dt, rows, cols, rng),
                                               vlt3.synthetic_blocks(dt, rows, cols, rng), dev)
        else:
            w = ops.QWeight.from_blocks(dt, rows, cols, vlt3.synthetic_blocks(dt, rows, cols, rng), dev)
        x = torch.randn(rows_in, cols, device=dev)
        y = torch.empty(rows_in, rows, device=dev)
        run = (lambda: ops.qlinear_swiglu(w, x, out=y)) if gu else (lambda: ops.qlinear(w, x, out=y))
        us = graph_time_us(run, 1, reps=reps)
        fl = 2.0 * rows_in * cols * rows * (2 if gu else 1)
        out.append({"proj": name, "dtype": "q4_0", "tokens": rows_in, "out": rows, "in": cols, "us": round(us, 1),
                    "tflops": round(fl / us / 1e6, 1), "frac": round(fl / us / 1e6 / 2500.0, 4)})
        del w
    return out


def _kv_copies(base, n: int):
    """n distinct versions of one set of KV span tensors (keys rotated by i, sign flipped for odd i), so
    that a round of calls reads n x the bytes and no call finds its KV in a cache."""
    import torch
    out = []
    for i in range(n):
        sgn = -1.0 if i & 1 else 1.0
        out.append([(sgn * torch.roll(k, i, dims=2), sgn * torch.roll(v, i, dims=2)) for k, v in base])
    return out


def attn_figures(dev, reps: int = 10):
    """Batched decode attention, bf16 KV: B=64, 12 q / 2 KV heads, D=128, keys 512 sink + 1024 segment
    + 2048 window = 3584; algorithmic bytes = K and V once (234,881,024 B) + q + out.  One graph replays
    a call over each of 2 KV copies (470 MB, beyond the 256 MB Infinity Cache); time per call."""
    import torch
    from vault_amd import ops
    B, H, G, D = 64, 12, 2, 128
    lens = (512, 1024, 1024, 1024)
    g = torch.Generator().manual_seed(11)
    base = [(torch.randn(B, G, n, D, generator=g).to(dev, torch.bfloat16),
             torch.randn(B, G, n, D, generator=g).to(dev, torch.bfloat16)) for n in lens]
    sets = _kv_copies(base, 2)
    q = torch.randn(B, H, D, generator=g).to(dev)
    out = torch.empty(B, H, D, device=dev)
    ws = ops.Workspace(dev)

    def run():
        for sp in sets:
            ops.attn_decode(q, sp, out=out, ws=ws)
    us = graph_time_us(run, len(sets), reps=reps)
    algo = B * sum(lens) * G * D * 2 * 2 + 2 * B * H * D * 4
    return {"config": "B=64 bf16 KV, 3584 keys (512 sink | 1024 seg | 2048 window)", "us": round(us, 2),
            "gbs": round(algo / us / 1e3, 1), "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 3)}


def attn_b1_figures(dev, reps: int = 20):
    """Single-layer decode attention, fp32 KV, batch 1: 12 q / 2 KV heads, D=128, keys 64 sink + 1024
    previous + 1024 current window = 2112; algorithmic bytes = K and V once (4,325,376 B) + q + out.
    One query per KV pair of rows, so the split launch and its merge launch are bound by latency, not
    by bandwidth.  One graph replays a call over each of 64 KV copies (277 MB, as the 28 layers of a
    decode step stream theirs); time per call (both launches)."""
    import torch
    from vault_amd import ops
    B, H, G, D = 1, 12, 2, 128
    lens = (64, 1024, 1024)
    g = torch.Generator().manual_seed(12)
    base = [(torch.randn(B, G, n, D, generator=g).to(dev), torch.randn(B, G, n, D, generator=g).to(dev))
            for n in lens]
    sets = _kv_copies(base, 64)
    q = torch.randn(B, H, D, generator=g).to(dev)
    out = torch.empty(B, H, D, device=dev)
    ws = ops.Workspace(dev)

    def run():
        for sp in sets:
            ops.attn_decode(q, sp, out=out, ws=ws)
    us = graph_time_us(run, len(sets), reps=reps)
    algo = B * sum(lens) * G * D * 4 * 2 + 2 * B * H * D * 4
    return {"config": "B=1 fp32 KV, 2112 keys (64 sink | 2048 window)", "us": round(us, 2),
            "gbs": round(algo / us / 1e3, 1), "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 3)}


def batched_decode(model, batch: int = 32, steps: int = 16, warmup: int = 4):
    """The same 1.54B model decoding 32 sequences at 100K context with bf16 KV (segment memory is off
    for batch > 1, as in the reference's batched path): tokens/s of the whole batch."""
    import torch
    from vault_amd.model import VAULTv3ForCausalLM
    m2 = VAULTv3ForCausalLM(model.w, kv_dtype=torch.bfloat16)
    st, _ = boundary_seeded_state(m2, batch, steps, warmup)
    dt = time_decode(m2, st, steps, warmup, batch)
    del st
    return {"config": f"batch {batch}, bf16 KV, 100K context (512 sinks + 2048 window), timed steps across "
                      f"the chunk boundary at 100,352",
            "tokens_per_s": round(batch * steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 3)}


CHAT_TOKENS = 16384
CHAT_KINDS = ("ids", "hop", "rollback", "clause", "words", "id")


def chat_prompt(cfg, toks, n_tokens: int = CHAT_TOKENS) -> list:
    """A multi-turn ChatML prompt of n_tokens: conversations (system line, a user turn of key / value
    lines, an assistant turn, a user question about earlier lines) back to back, ~150 tokens each, so
    that user turns end in every 1024-token chunk; it ends with a question and the assistant header."""
    from tests import modelgen
    ids, i = [], 0
    while True:
        conv = modelgen.conversation(cfg, toks, CHAT_KINDS[i % len(CHAT_KINDS)], seed=i, answer=20)
        if len(ids) + len(conv) - 20 >= n_tokens:
            q = modelgen.conversation(cfg, toks, "ids", seed=i, answer=0)
            return ids[:n_tokens - len(q)] + q
        ids += conv
        i += 1


def prefill_model_figures(model, L: int = 8192, reps: int = 3):
    """model.prefill of an L-token prompt of random ids (batch 1, the chunk-recurrent path with segment
    memory: chunk GEMMs on the tiled kernel, MFMA chunk attention, the boundary's bank merge), fp32 KV
    (the model's state) and bf16 KV; tokens/s as the median of ``reps`` timed prefills after a warm-up."""
    import torch
    from vault_amd.model import VAULTv3ForCausalLM
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(0, model.cfg.vocab_size, (1, L), generator=g)
    out = {"config": f"model.prefill, batch 1, {L} random ids, segment memory on"}
    for name, kv in (("fp32_kv", torch.float32), ("bf16_kv", torch.bfloat16)):
        m = model if kv == model.kv_dtype else VAULTv3ForCausalLM(model.w, kv_dtype=kv)
        m.prefill(ids[:, :2048])
        ts = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            m.prefill(ids)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        out[f"{name}_tokens_per_s"] = round(L / sorted(ts)[len(ts) // 2], 1)
    return out


def chat_figures(model, decode_steps: int = 48):
    """The 1.54B model with token strings (a synthetic word vocabulary over the 151665 ids: ChatML
    specials, key / value words, break-tier punctuation), so the resonance, quarantine and segment
    rules all run: a CHAT_TOKENS-token multi-turn ChatML prefill (batch 1, fp32 KV, segment memory
    on), then decode_steps greedy steps fed by host ids (the logits' argmax read on the host) and,
    after the same prefill again, fed by device ids (ops.argmax).  Reports prefill tokens/s, the
    chunks whose attention carried a resonance bias, and per-step decode rates (medians, each step
    timed between synchronisations) of the steps with the resonance bias on and of the others."""
    import copy
    import torch
    from tests import modelgen
    from vault_amd import ops
    from vault_amd.model import VAULTv3ForCausalLM
    from vault_amd.tokens import TokenTable
    cfg = model.cfg
    toks, bmap = modelgen.word_vocab(cfg)
    w = copy.copy(model.w)
    w.tokens = TokenTable(toks, bmap, cfg.vocab_size)
    m = VAULTv3ForCausalLM(w, kv_dtype=torch.float32)
    ids = torch.tensor([chat_prompt(cfg, toks)])
    biased = []
    chunk_bias = m._chunk_bias

    def counted(*a, **k):
        r = chunk_bias(*a, **k)
        biased.append(r is not None)
        return r

    m._chunk_bias = counted
    m.prefill(ids[:, :2048])                          # warm-up (library loads, workspaces)
    out = {"config": f"{ids.shape[1]}-token multi-turn ChatML prompt, batch 1, fp32 KV, segment memory on, "
                     f"token strings (resonance / quarantine rules active)"}
    for leg in ("host_ids", "device_ids"):
        biased.clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        last, st = m.prefill(ids)
        torch.cuda.synchronize()
        t_pre = time.perf_counter() - t0
        if leg == "host_ids":
            out["prefill_tokens_per_s"] = round(ids.shape[1] / t_pre, 1)
            out["prefill_chunks_biased"] = f"{sum(biased)} of {len(biased)}"
        tok = torch.tensor([int(last[0].argmax())]) if leg == "host_ids" else ops.argmax(last)
        times = {True: [], False: []}
        for _ in range(decode_steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            logits = m.step(tok, st)
            tok = torch.tensor([int(logits[0].argmax())]) if leg == "host_ids" else ops.argmax(logits)
            torch.cuda.synchronize()
            times[st.seg_bias_mode > 0].append(time.perf_counter() - t0)
        # medians: the first step of each graph configuration captures it (an outlier, not a rate)
        for on, name in ((True, "resonating"), (False, "quiet")):
            t = sorted(times[on])
            out[f"decode_{leg}_{name}_steps"] = len(t)
            if t:
                out[f"decode_{leg}_{name}_tokens_per_s"] = round(1.0 / t[len(t) // 2], 1)
    return out


PREFILL_FLOPS = 90.22e9   # unmasked (query, key) pairs x 4 x D x H for L = 8192, W = 1024, 512 sinks


def prefill_figures(dev, reps: int = 10):
    """Block sliding-window attention prefill, bf16: batch 1, L = 8192, 12 q / 2 kv heads, D = 128,
    W = 1024, 512 sinks re-rotated per chunk (drop-in block_sliding_attention: 6 sink re-rotations + one
    MFMA attention launch over the 8 chunks).  Algorithmic work: 4 D H flops per visible (query, key)
    pair = 90.22 GFLOP; peak 2.5 PFLOP/s dense bf16."""
    import torch
    from vault_amd import attention as vatt
    B, H, G, D, L, W, S = 1, 12, 2, 128, 8192, 1024, 512
    g = torch.Generator().manual_seed(13)
    q, k, v, kr = (torch.randn(B, n, L, D, generator=g).to(dev, torch.bfloat16) for n in (H, G, G, G))
    run = lambda: vatt.block_sliding_attention(q, k, v, W, k_raw=kr, n_sink=S, head_dim=D, rope_theta=1e6)
    run()
    torch.cuda.synchronize()
    e0, e1 = _events()
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    tf = PREFILL_FLOPS / us / 1e6
    return {"config": "bf16 L=8192 W=1024 sinks=512 12q/2kv D=128", "us": round(us, 1), "tflops": round(tf, 1),
            "frac": round(tf / 2500.0, 4)}


def cpu_baseline(cfg, tensors, budget_s: float = 15.0):
    """The reference C runtime (runtime/vault3.c, compiled into oracle/_ref) stepping the same model
    from a state seeded at the same context position, on the host's cores."""
    from oracle import ref
    from vault_amd import vlt3
    if not ref.available():
        return None
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.vlt3")
        vlt3.write_vlt3(path, list(tensors.values()), cfg, vlt3.Q4_0)
        with open(path, "rb") as f:
            image = f.read()
    rt = ref.RefRuntime(image, threads=threads, verify=False)
    del image
    # Like the GPU leg, the timed steps cross the chunk boundary at 100,352 (segment-bank merge,
    # compaction, ring swap, re-rotations): the first timed step decodes position 100,352 - 100.
    W = cfg.window
    b2 = (CTX_POS // W + 1) * W
    p_first = b2 - 100
    rt.seed_long_context(p_first - 1, N_PIN, MEM_CNT, seed=3)
    rt.step(1)
    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0 < budget_s or n <= 100) and n < 300:
        rt.step(2 + n)
        n += 1
    dt = time.perf_counter() - t0
    assert rt.info()["pos"] > b2, "the timed steps did not reach the chunk boundary"
    rt.close()
    return {"value": round(n / dt, 3), "unit": "tokens/s", "cores": threads, "host_cores": os.cpu_count(),
            "host_cores_usable": len(os.sched_getaffinity(0)), "kind": "reference",
            "sample": f"{n} decode steps of the same 1.54B hybrid-Q4_0 model from position {p_first}, across "
                      f"the chunk boundary at {b2} (512 sinks, 1024 segment slots, fp32 state) with "
                      f"runtime/vault3.c v3_step, "
                      f"{threads} threads on a host with {os.cpu_count()} cores ({len(os.sched_getaffinity(0))} "
                      f"usable by this process)"}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "traffic_attn_decode_fp32_b1_3584.md")
COPY_BYTES = 256 << 20      # calibration stream for the PMC byte counters (read and written once)


def pmc_launches(dev, rounds: int = 4) -> None:
    """The launches the PMC runs count: the roofline call (attention + merge) eagerly over the
    ATTN_COPIES KV copies (``rounds`` times) and a plain streaming kernel that reads and writes
    COPY_BYTES once (torch's elementwise negation, a name no other launch here has), ``rounds`` times."""
    import torch
    from vault_amd import ops
    B, H, G, D = 1, 12, 2, 128
    g = torch.Generator().manual_seed(12)
    base = [(torch.randn(B, G, n, D, generator=g).to(dev), torch.randn(B, G, n, D, generator=g).to(dev))
            for n in ATTN_LENS]
    sets = _kv_copies(base, ATTN_COPIES)
    q = torch.randn(B, H, D, generator=g).to(dev)
    out = torch.empty(B, H, D, device=dev)
    ws = ops.Workspace(dev)
    src = torch.randn(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(rounds):
        for sp in sets:
            ops.attn_decode(q, sp, out=out, ws=ws)
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    _log(f"pmc launches done: {rounds} x {len(sets)} attention calls, {rounds} streams of {COPY_BYTES} B")


def _pmc_avg(csv_path: str, counter: str, name_part: str) -> tuple[float, int]:
    import csv
    vals = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter and name_part in r["Kernel_Name"]:
                vals.append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit(f"{csv_path}: no {counter} rows for kernels matching {name_part!r}")
    return sum(vals) / len(vals), len(vals)


def pmc_report(fetch_csv: str, write_csv: str) -> None:
    """Markdown summary of the two PMC runs: per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the two
    kernels of the roofline call and of the calibration copy, the copy's bytes / counter factor, and
    the scaled HBM traffic per call (the figure ``roofline.traffic`` reports)."""
    kerns = (("attn_decode_b1_kernel<0, 6, 8, 2, 0, true>", "split attention"), ("b1_merge_kernel", "split merge"))
    copy = "neg_kernel"
    fc, nc = _pmc_avg(fetch_csv, "FETCH_SIZE", copy)
    wc, _ = _pmc_avg(write_csv, "WRITE_SIZE", copy)
    f_scale, w_scale = COPY_BYTES / (fc * 1024), COPY_BYTES / (wc * 1024)
    rows, traffic = [], 0.0
    for name, what in kerns:
        fk, nk = _pmc_avg(fetch_csv, "FETCH_SIZE", name)
        wk, _ = _pmc_avg(write_csv, "WRITE_SIZE", name)
        traffic += fk * 1024 * f_scale + wk * 1024 * w_scale
        rows.append(f"| {nk} | `{name}` ({what}) | {fk:.1f} | {wk:.1f} |")
    algo = ATTN_ALGO_BYTES
    print("| dispatches | kernel | FETCH_SIZE KiB | WRITE_SIZE KiB |\n|---|---|---|---|\n" + "\n".join(rows) + "\n"
          f"| {nc} | torch `neg` elementwise kernel ({COPY_BYTES} B read + written) | {fc:.1f} | {wc:.1f} |\n\n"
          f"copy calibration: fetch factor {f_scale:.4f}, write factor {w_scale:.4f} (bytes / (KiB x 1024))\n\n"
          f"algorithmic bytes per call: {algo}\n\n"
          f"traffic_bytes_per_launch: {traffic:.0f}\n\n"
          f"traffic / algorithmic: {traffic / algo:.3f}")


def measured_traffic():
    """HBM bytes per call of the roofline kernels from the committed PMC summary, or None."""
    import re
    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"traffic_bytes_per_launch: (\d+)", f.read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--kv", choices=("fp32", "bf16"), default="fp32")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-kernels", action="store_true", help="skip the secondary kernel figures")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the timed decode steps (for per-kernel profiles of the step)")
    ap.add_argument("--figures", choices=("gemv", "attn_decode", "attn_decode_b1", "attn_prefill", "gemm_prefill",
                                          "roofline", "gateup", "decode_batch32", "lm_head", "chat",
                                          "prefill_model"),
                    help="only one set of kernel figures, printed as JSON (for per-kernel profiles)")
    ap.add_argument("--pmc", action="store_true",
                    help="only run the launches the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs count")
    ap.add_argument("--pmc-report", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 counter_collection.csv files (no GPU needed)")
    args = ap.parse_args()
    if args.pmc_report:
        pmc_report(*args.pmc_report)
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (decode shards by "
              "independent sequences with no exchange); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from vault_amd import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    if args.pmc:
        pmc_launches(dev)
        return 0
    if args.figures == "roofline":
        # the roofline measurement of the default run alone (its launches, for a kernel trace)
        print(json.dumps({"roofline": attention_kernel(dev)}), flush=True)
        return 0
    if args.figures == "gateup":
        cfg = model_config()
        model, tensors = build_model(cfg, dev, torch.float32)
        del tensors
        print(json.dumps({"gateup_gemv": gateup_kernel(model)}), flush=True)
        return 0
    if args.figures == "decode_batch32":
        cfg = model_config()
        model, tensors = build_model(cfg, dev, torch.float32)
        del tensors
        print(json.dumps({"decode_batch32": batched_decode(model)}), flush=True)
        return 0
    if args.figures == "chat":
        cfg = model_config()
        model, tensors = build_model(cfg, dev, torch.float32)
        del tensors
        print(json.dumps({"chat": chat_figures(model)}), flush=True)
        return 0
    if args.figures == "prefill_model":
        cfg = model_config()
        model, tensors = build_model(cfg, dev, torch.float32)
        del tensors
        print(json.dumps({"prefill_model": prefill_model_figures(model)}), flush=True)
        return 0
    if args.figures == "lm_head":
        # the 151665 x 1536 rows of the gemv figures at batch 1 (for the streaming kernel's profiles)
        print(json.dumps({"lm_head": gemv_figures(dev, batches=(1,), shapes=[(151665, 1536)])}), flush=True)
        return 0
    if args.figures:
        fig = {"gemv": gemv_figures, "attn_decode": attn_figures, "attn_decode_b1": attn_b1_figures,
               "attn_prefill": prefill_figures,
               "gemm_prefill": gemm_figures}[args.figures](dev)
        print(json.dumps({args.figures: fig}), flush=True)
        return 0
    kv_dtype = torch.float32 if args.kv == "fp32" else torch.bfloat16
    cfg = model_config()
    model, tensors = build_model(cfg, dev, kv_dtype)
    st, p0 = boundary_seeded_state(model, args.batch, args.steps, args.warmup)
    _log(f"model and state ready (state {st.nbytes() / 2**20:.0f} MiB); timing {args.steps} steps from "
         f"position {p0 + args.warmup}")
    dt = time_decode(model, st, args.steps, args.warmup, args.batch)
    tok_s = args.batch * args.steps / dt
    ms = dt * 1e3 / args.steps
    _log(f"decode: {tok_s:.1f} tokens/s ({ms:.3f} ms/step)")

    if args.decode_only:
        print(json.dumps({"metric": "decode tokens/s (decode-only profile run)", "value": round(tok_s, 2),
                          "unit": "tokens/s", "ms_per_step": round(ms, 4), "steps": args.steps}), flush=True)
        return 0
    dom = attention_kernel(dev)
    _log(f"roofline kernel (attention + merge): {dom['avg_us']:.2f} us, {dom['gbs']:.0f} GB/s")
    kernels = {"gateup_gemv": gateup_kernel(model), "copy_peak": copy_peak(dev)}
    if not args.no_kernels:
        kernels["gemv"] = gemv_figures(dev)
        kernels["attn_decode"] = attn_figures(dev)
        kernels["attn_decode_b1"] = attn_b1_figures(dev)
        kernels["attn_prefill"] = prefill_figures(dev)
        kernels["gemm_prefill"] = gemm_figures(dev)
        if args.batch == 1:
            kernels["decode_batch32"] = batched_decode(model)
            kernels["prefill_8192"] = prefill_model_figures(model)
            kernels["chat"] = chat_figures(model)
        _log("kernel figures done")
    cpu = None
    if not args.no_cpu and args.batch == 1 and args.kv == "fp32":
        cpu = cpu_baseline(cfg, tensors)
        if cpu:
            _log(f"cpu baseline: {cpu['value']} tokens/s on {cpu['cores']} threads")

    # algorithmic bytes of one decode step (weights + LM head + scorer + KV read)
    timed = range(p0 + args.warmup, p0 + args.warmup + args.steps)
    n_keys_avg = N_PIN + (MEM_CNT if args.batch == 1 else 0) + cfg.window + \
        sum(p % cfg.window + 1 for p in timed) / max(1, args.steps)
    kv_bytes = cfg.n_layers * n_keys_avg * 2 * cfg.head_dim * 2 * (4 if args.kv == "fp32" else 2) * args.batch
    step_bytes = model.w.layer_stream_bytes() + model.w.embed.stream_bytes + kv_bytes + \
        (model.w.scorer.w1.stream_bytes if (model.w.scorer is not None and args.batch == 1) else 0)
    line = {
        "metric": "decode tokens/s, 1.54B hybrid-Q4_0 @100K ctx (with decode attn + Q8/Q4 GEMV GB/s)",
        "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if args.kv == "fp32" else "f32 (bf16 KV)", "data": "synthetic (seeded random-init weights as quantized blocks, seeded KV state)",
        "config": {"workload": "28-layer 1.54B hybrid-Q4_0 decode step at 100K context (512 sinks, 1024 segment KV, "
                               "2048 window, segment scorer on), timed steps across the chunk boundary at 100,352",
                   "batch": args.batch, "context": p0 + args.warmup,
                   "kv_dtype": args.kv, "parallelism": "single GPU"},
        "step_gbs": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(dom["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": dom["kernel"], "avg_us": round(dom["avg_us"], 3),
                     "bytes_per_launch": dom["bytes_per_launch"], "cache_resident_us": dom["cache_resident_us"]},
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
