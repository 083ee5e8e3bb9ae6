"""Full-size parity of the reference's "bf16" weight format (tools/vlt3.py:312-330: BF16 embedding
and projections, F32 norms, biases and scorer): the 28-layer random-init 1.54B model written by this
repo's VLT3 writer, loaded through the drop-in loader (ModelWeights.from_vlt3: validation, device
NaN / Inf scan, packing of the BF16 rows), decoding at 100K-token context against the reference C
runtime (runtime/vault3.c, whose row_dot widens BF16 to fp32, :510-525) on the identical seeded state.
Bars as for the hybrid-Q4_0 model: rel < 1e-4, max|dlogit| <= 5e-2, 100% top-1, identical
segment-memory slots after the chunk boundary; batch 16 (the fp32 MFMA GEMM over BF16 weights,
including the LM head) against the runtime stepping each sequence alone.
"""
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import ref
from tests.test_gpu_fullsize import N_PIN, MEM_CNT, _compare, _seed_both
from vault_amd import vlt3
from vault_amd.config import QWEN25_1P5B
from vault_amd.model import VAULTv3ForCausalLM
from vault_amd.weights import ModelWeights, synthetic_tensors

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")]


@pytest.fixture(scope="module")
def bf16_model(dev):
    from dataclasses import replace
    cfg = replace(QWEN25_1P5B, vocab_size=151665, auto_pin_system=False)
    tensors = synthetic_tensors(cfg, "bf16", 4321)
    assert tensors["layers.3.mlp.down_proj.weight"].dtype == vlt3.BF16
    assert tensors["embed_tokens.weight"].dtype == vlt3.BF16
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.vlt3")
        vlt3.write_vlt3(path, list(tensors.values()), cfg, vlt3.BF16)
        del tensors
        print("bf16 model written", flush=True)
        w = ModelWeights.from_vlt3(path, dev)
        with open(path, "rb") as f:
            image = f.read()
    print("bf16 model loaded", flush=True)
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    rt = ref.RefRuntime(image, threads=threads, verify=False)
    del image
    m = VAULTv3ForCausalLM(w, kv_dtype=torch.float32)
    yield w.cfg, m, rt
    rt.close()


def test_bf16_decode_at_100k_matches_reference_runtime(bf16_model):
    cfg, m, rt = bf16_model
    st = _seed_both(cfg, m, rt, 100_000)
    _compare(m, rt, st, np.random.default_rng(15).integers(0, cfg.vocab_size, 4))


def test_bf16_decode_across_chunk_boundary_matches_reference_runtime(bf16_model):
    cfg, m, rt = bf16_model
    st = _seed_both(cfg, m, rt, 100_349)
    _compare(m, rt, st, np.random.default_rng(16).integers(0, cfg.vocab_size, 5))
    assert np.array_equal(rt.mem_pos(), st.mem_pos.numpy())


def test_bf16_batch16_decode_matches_reference_runtime(bf16_model):
    """16 sequences without segment memory (the reference's batched path) at 100,350 .. 100,352."""
    from tests.test_gpu_fullsize import _seed_batch_and_reference
    import tests.test_gpu_fullsize as fs
    cfg, m, rt = bf16_model
    B = 16
    ids = np.random.default_rng(17).integers(0, cfg.vocab_size, (B, 3))
    old = fs.BATCH
    fs.BATCH = B
    try:
        st, want = _seed_batch_and_reference(cfg, m, rt, 100_350, ids, torch.float32)
    finally:
        fs.BATCH = old
    for i in range(ids.shape[1]):
        got = m.step(torch.from_numpy(ids[:, i]), st).double().cpu().numpy()
        w = want[:, i].astype(np.float64)
        rel = np.abs(got - w).max(axis=1) / np.abs(w).max(axis=1)
        print(f"batch 16 bf16 step {i}: worst rel {float(rel.max()):.3e}", flush=True)
        assert rel.max() < 1e-4, (i, float(rel.max()))
        assert np.array_equal(got.argmax(1), w.argmax(1)), i
