"""VAULTv3Config: the hyper-parameters of the reference model (src/vault_v3_model.py:37-103),
same field names and defaults, plus the VLT3 header mapping (docs/VAULT_v3_SPEC.md:111-136)."""
from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Tuple


@dataclass
class VAULTv3Config:
    vocab_size: int = 151936
    d_model: int = 1536
    n_layers: int = 28
    n_heads: int = 12
    n_kv_heads: int = 2
    head_dim: int = 128
    d_ff: int = 8960
    rms_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    tie_embeddings: bool = True
    window: int = 1024
    n_sink: int = 4
    max_sink: int = 512
    auto_pin_system: bool = True
    im_start_id: int = 151644
    im_end_id: int = 151645
    system_tok_id: int = 8948
    seg_budget: int = 0
    seg_hidden: int = 256
    seg_min: int = 16
    seg_max: int = 48
    seg_layers: Tuple[int, ...] = ()

    @property
    def group_size(self) -> int:
        return self.n_heads // self.n_kv_heads

    @property
    def has_seg_scorer(self) -> bool:
        return len(self.seg_layers) > 0 and self.seg_budget > 0

    @property
    def sink_cap(self) -> int:
        """Sink slots of the state (src/vault_v3_model.py:964)."""
        return max(1, self.n_sink, self.max_sink if self.auto_pin_system else self.n_sink)

    def to_dict(self) -> dict:
        d = asdict(self)
        d["seg_layers"] = list(self.seg_layers)
        return d

    @classmethod
    def from_dict(cls, d: dict) -> "VAULTv3Config":
        d = {k: v for k, v in dict(d).items() if k in cls.__dataclass_fields__}
        if "seg_layers" in d:
            d["seg_layers"] = tuple(int(x) for x in d["seg_layers"])
        return cls(**d)

    @classmethod
    def from_vlt3_header(cls, h: dict) -> "VAULTv3Config":
        nf = h.get("seg_n_feat", 0)
        return cls(
            vocab_size=h["vocab_size"], d_model=h["d_model"], n_layers=h["n_layers"], n_heads=h["n_heads"],
            n_kv_heads=h["n_kv_heads"], head_dim=h["head_dim"], d_ff=h["d_ff"], rms_eps=h["rms_eps"],
            rope_theta=h["rope_theta"], tie_embeddings=bool(h["flags"] & 1), window=h["window"], n_sink=h["n_sink"],
            seg_budget=h["seg_budget"] if nf else 0, seg_hidden=h["seg_hidden"] if nf else 256,
            seg_min=h["seg_min"] if nf else 16, seg_max=h["seg_max"] if nf else 48,
            seg_layers=tuple(h[f"seg_layer{i}"] for i in range(nf)) if nf else (),
            im_start_id=h["im_start_id"], im_end_id=h["im_end_id"],
        )


QWEN25_1P5B = VAULTv3Config(window=1024, n_sink=512, max_sink=512, seg_budget=1024, seg_hidden=256, seg_min=16,
                            seg_max=48, seg_layers=(8, 16, 24))
