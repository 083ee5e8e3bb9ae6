"""Model weights on the device: every projection as a packed QWeight, norms / biases as fp32.

Projections that share a dtype are fused into one packed tensor so that one GEMV launch streams
them: q|k|v when all three share a dtype (else q alone and k|v), and gate/up interleaved for the
SwiGLU epilogue.  The tied LM head reuses the embedding tensor (src/vault_v3_model.py:2150-2151).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np
import torch

from . import ops, vlt3
from .config import VAULTv3Config
from .tokens import TokenTable

Tensor = vlt3.Tensor


@dataclass
class LayerWeights:
    ln1: torch.Tensor
    ln2: torch.Tensor
    wq: Optional[ops.QWeight]        # None when fused into wqkv
    wqkv: ops.QWeight                # q|k|v fused, or k|v when q is separate
    bq: torch.Tensor
    bqkv: torch.Tensor               # bias matching wqkv's rows
    wo: ops.QWeight
    wgu: ops.QWeight
    wd: ops.QWeight
    wq_rope: Optional[ops.QWeight] = None    # q rows in RoPE-pair order (one-token decode kernel)
    wkv_rope: Optional[ops.QWeight] = None   # k rows in RoPE-pair order, then v rows


@dataclass
class ScorerWeights:
    ln_w: torch.Tensor
    ln_b: torch.Tensor
    w1: ops.QWeight
    b1: torch.Tensor
    w2: torch.Tensor   # [hidden] fp32
    b2: torch.Tensor   # [1]


def _f32(t: Tensor, device, uploaded: Optional[torch.Tensor] = None) -> torch.Tensor:
    """An F32 tensor as fp32 on the device: the uploaded payload viewed as floats, or a fresh upload."""
    if t.dtype != vlt3.F32:
        raise vlt3.VLT3Error(f"{t.name} must be F32")
    if uploaded is not None:
        return uploaded.view(torch.float32)
    return torch.from_numpy(np.frombuffer(t.data, dtype="<f4").copy()).to(device)


def _block_dtype(t: Tensor) -> int:
    """Projection weights: Q8_0 / Q4_0 blocks, or F32 / BF16 / F16 elements (runtime/vault3.c:499-598)."""
    if t.dtype not in (vlt3.Q8_0, vlt3.Q4_0, vlt3.F32, vlt3.BF16, vlt3.F16):
        raise vlt3.VLT3Error(f"{t.name}: dtype {t.dtype} is not supported on the device path")
    if t.shape[-1] % 32:
        raise vlt3.VLT3Error(f"{t.name}: rows of {t.shape[-1]} elements are not whole 32-element blocks")
    return t.dtype


class ModelWeights:
    def __init__(self, cfg: VAULTv3Config, device):
        self.cfg = cfg
        self.device = torch.device(device)
        self.layers: List[LayerWeights] = []
        self.embed: Optional[ops.QWeight] = None
        self.norm: Optional[torch.Tensor] = None
        self.scorer: Optional[ScorerWeights] = None
        # token strings (VTOK) when known: break tiers, system-role and newline rules of the driver
        self.tokens: Optional[TokenTable] = None

    # ------------------------------------------------------------------ construction
    @classmethod
    def from_tensors(cls, cfg: VAULTv3Config, tensors: Dict[str, Tensor], device,
                     tokens: Optional[TokenTable] = None, scan: bool = True) -> "ModelWeights":
        """Upload and pack every tensor.  ``scan``: reject non-finite weights and block scales on the
        device first (the reference loader's NaN / Inf rule, runtime/vault3.c:215-271)."""
        self = cls(cfg, device)
        self.tokens = tokens
        dev = self.device
        # every payload crosses the bus once: the scan and the packing kernels read the same upload
        up = {n: ops.QWeight._upload(t.data, dev) for n, t in tensors.items()}
        if scan:
            bad = ops.count_nonfinite([(t.dtype, up[n], int(np.prod(t.shape))) for n, t in tensors.items()], dev)
            if any(bad):
                names = [n for n, k in zip(tensors, bad) if k]
                e = vlt3.VLT3Error(f"non-finite weights or scales in {names[:4]}")
                e.code = vlt3.E_NAN
                raise e
        f32 = lambda name: _f32(tensors[name], dev, up[name])
        emb = tensors["embed_tokens.weight"]
        self.embed = ops.QWeight.from_blocks(_block_dtype(emb), cfg.vocab_size, cfg.d_model, up["embed_tokens.weight"],
                                             dev)
        self.norm = f32("norm.weight")
        H, G, D, d, F = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.d_model, cfg.d_ff
        for li in range(cfg.n_layers):
            p = f"layers.{li}."
            t = {k[len(p):]: v for k, v in tensors.items() if k.startswith(p)}
            u_ = lambda n: up[p + n]
            q, k, v = t["self_attn.q_proj.weight"], t["self_attn.k_proj.weight"], t["self_attn.v_proj.weight"]
            bq, bk, bv = (f32(f"{p}self_attn.{n}_proj.bias") for n in "qkv")
            kv_data = torch.cat([u_("self_attn.k_proj.weight"), u_("self_attn.v_proj.weight")])
            if _block_dtype(q) == _block_dtype(k) == _block_dtype(v):
                wq = None
                wqkv = ops.QWeight.from_blocks(q.dtype, H * D + 2 * G * D, d,
                                               torch.cat([u_("self_attn.q_proj.weight"), kv_data]), dev)
                bqkv = torch.cat([bq, bk, bv])
            else:
                if _block_dtype(k) != _block_dtype(v):
                    raise vlt3.VLT3Error("k_proj and v_proj must share a dtype")
                wq = ops.QWeight.from_blocks(q.dtype, H * D, d, u_("self_attn.q_proj.weight"), dev)
                wqkv = ops.QWeight.from_blocks(k.dtype, 2 * G * D, d, kv_data, dev)
                bqkv = torch.cat([bk, bv])
            wq_rope = ops.QWeight.rope_from_blocks(q.dtype, H * D, d, u_("self_attn.q_proj.weight"), D, H * D, dev)
            wkv_rope = ops.QWeight.rope_from_blocks(k.dtype, 2 * G * D, d, kv_data, D, G * D, dev)
            o = t["self_attn.o_proj.weight"]
            g, u, dn = t["mlp.gate_proj.weight"], t["mlp.up_proj.weight"], t["mlp.down_proj.weight"]
            if _block_dtype(g) != _block_dtype(u):
                raise vlt3.VLT3Error("gate_proj and up_proj must share a dtype")
            self.layers.append(LayerWeights(
                ln1=f32(p + "input_layernorm.weight"), ln2=f32(p + "post_attention_layernorm.weight"),
                wq=wq, wqkv=wqkv, bq=bq, bqkv=bqkv,
                wo=ops.QWeight.from_blocks(_block_dtype(o), d, H * D, u_("self_attn.o_proj.weight"), dev),
                wgu=ops.QWeight.gateup_from_blocks(g.dtype, F, d, u_("mlp.gate_proj.weight"), u_("mlp.up_proj.weight"),
                                                   dev),
                wd=ops.QWeight.from_blocks(_block_dtype(dn), d, F, u_("mlp.down_proj.weight"), dev),
                wq_rope=wq_rope, wkv_rope=wkv_rope,
            ))
        if cfg.has_seg_scorer and "seg_scorer.ln.weight" in tensors:
            fd = len(cfg.seg_layers) * d
            w2 = f32("seg_scorer.fc2.weight")
            self.scorer = ScorerWeights(
                ln_w=f32("seg_scorer.ln.weight"), ln_b=f32("seg_scorer.ln.bias"),
                w1=ops.QWeight.from_blocks(vlt3.F32, cfg.seg_hidden, fd, up["seg_scorer.fc1.weight"], dev),
                b1=f32("seg_scorer.fc1.bias"), w2=w2.reshape(-1),
                b2=f32("seg_scorer.fc2.bias"))
        torch.cuda.synchronize(dev)
        return self

    @classmethod
    def from_vlt3(cls, path: str, device, check_crc: bool = True) -> "ModelWeights":
        """Load a VLT3 file: host validation (``vlt3.read_vlt3``), then upload with the device NaN /
        Inf scan; the file's VTOK token strings drive the break tiers and the auto-pin rules."""
        vf = vlt3.read_vlt3(path, check_crc=check_crc)
        cfg = VAULTv3Config.from_vlt3_header(vf.header)
        return cls.from_tensors(cfg, vf.tensors, device, tokens=vf.tokens)

    # ------------------------------------------------------------------ accounting
    def layer_stream_bytes(self) -> int:
        tot = 0
        for lw in self.layers:
            for w in (lw.wq, lw.wqkv, lw.wo, lw.wgu, lw.wd):
                if w is not None:
                    tot += w.stream_bytes
        return tot


# ----------------------------------------------------------------------------------------------
# tensor sets (quantized per the hybrid policy, or drawn directly as quantized blocks)
# ----------------------------------------------------------------------------------------------

def tensor_shapes(cfg: VAULTv3Config) -> Dict[str, tuple]:
    H, G, D, d, F = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.d_model, cfg.d_ff
    s = {"embed_tokens.weight": (cfg.vocab_size, d), "norm.weight": (d,)}
    for li in range(cfg.n_layers):
        p = f"layers.{li}."
        s.update({
            p + "input_layernorm.weight": (d,), p + "self_attn.q_proj.weight": (H * D, d), p + "self_attn.q_proj.bias": (H * D,),
            p + "self_attn.k_proj.weight": (G * D, d), p + "self_attn.k_proj.bias": (G * D,),
            p + "self_attn.v_proj.weight": (G * D, d), p + "self_attn.v_proj.bias": (G * D,),
            p + "self_attn.o_proj.weight": (d, H * D), p + "post_attention_layernorm.weight": (d,),
            p + "mlp.gate_proj.weight": (F, d), p + "mlp.up_proj.weight": (F, d), p + "mlp.down_proj.weight": (d, F),
        })
    if cfg.has_seg_scorer:
        fd = len(cfg.seg_layers) * d
        s.update({"seg_scorer.ln.weight": (fd,), "seg_scorer.ln.bias": (fd,), "seg_scorer.fc1.weight": (cfg.seg_hidden, fd),
                  "seg_scorer.fc1.bias": (cfg.seg_hidden,), "seg_scorer.fc2.weight": (1, cfg.seg_hidden),
                  "seg_scorer.fc2.bias": (1,)})
    return s


def quantize_state(cfg: VAULTv3Config, state: Dict[str, np.ndarray], fmt: str) -> Dict[str, Tensor]:
    """fp32 arrays -> VLT3 tensors with the hybrid dtype policy (tools/vlt3.py:312-330)."""
    out = {}
    for name, arr in state.items():
        dt = vlt3.choose_dtype(name, fmt, cfg.n_layers)
        a = np.asarray(arr, dtype=np.float32)
        if dt in (vlt3.Q8_0, vlt3.Q4_0) and a.shape[-1] % 32:
            dt = vlt3.BF16                       # rows that are not whole blocks (tools/vlt3.py:341-342)
        out[name] = Tensor(name, dt, tuple(a.shape), vlt3.quantize(dt, a))
    return out


def random_state(cfg: VAULTv3Config, seed: int, std: float = 0.15) -> Dict[str, np.ndarray]:
    """fp32 random-init weights in the recipe of the reference's runtime tests
    (tests/test_vlt3_runtime.py:33-49): norms U(0.8, 1.2), scorer LN bias N(0, 0.05), else N(0, std)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shp in tensor_shapes(cfg).items():
        if "layernorm" in name or name in ("norm.weight", "seg_scorer.ln.weight"):
            out[name] = rng.uniform(0.8, 1.2, shp).astype(np.float32)
        elif name == "seg_scorer.ln.bias":
            out[name] = (rng.standard_normal(shp) * 0.05).astype(np.float32)
        else:
            out[name] = (rng.standard_normal(shp) * std).astype(np.float32)
    return out


def synthetic_tensors(cfg: VAULTv3Config, fmt: str, seed: int) -> Dict[str, Tensor]:
    """Random-init weights drawn directly as quantized blocks (hybrid policy; BF16 projections
    N(0, 0.02) for the "bf16" format), F32 norms U(0.8,1.2), biases N(0, 0.02), scorer fp32 N(0, 0.02):
    the synthetic recipe of the 1.54B decode workload."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shp in tensor_shapes(cfg).items():
        dt = vlt3.choose_dtype(name, fmt, cfg.n_layers)
        if dt in (vlt3.Q8_0, vlt3.Q4_0):
            out[name] = Tensor(name, dt, shp, vlt3.synthetic_blocks(dt, shp[0], shp[1], rng))
            continue
        if dt in (vlt3.BF16, vlt3.F16):
            a = rng.standard_normal(shp, dtype=np.float32) * np.float32(0.02)
            out[name] = Tensor(name, dt, shp, vlt3.quantize(dt, a))
            continue
        if "layernorm" in name or name in ("norm.weight", "seg_scorer.ln.weight"):
            a = rng.uniform(0.8, 1.2, shp).astype(np.float32)
        else:
            a = (rng.standard_normal(shp) * 0.02).astype(np.float32)
        out[name] = Tensor(name, vlt3.F32, shp, a.astype("<f4").tobytes())
    return out
