"""vault_amd: MI355X (gfx950) implementation of the VAULT v3 decode/prefill hot path.

Block sliding-window GQA attention over [sink | segment memory | rolling window] with RoPE, and
the Q8_0 / hybrid-Q4_0 block-dequant GEMV/GEMM of every projection, as hand-written HIP kernels
behind a C ABI (include/vault_amd.h), driven from a Python ``prefill()`` / ``step()`` host that
mirrors ``VAULTv3ForCausalLM`` (src/vault_v3_model.py:2153-2311).
"""

__version__ = "0.1.0"
