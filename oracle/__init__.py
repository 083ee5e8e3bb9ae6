"""CPU oracle for the VAULT v3 decode/prefill hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``vault_amd`` imports this package; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only to check results (never as the thing measured or
shipped).

Contents (each function cites the reference file:line it restates):

* ``codec``     Q8_0 / Q4_0 block decode (tools/vlt3.py:98-157), fp16 decode.
* ``linalg``    fp64-accumulated GEMV / SwiGLU / RMSNorm (runtime/vault3.c:499-660).
* ``rope``      RoPE tables in the C runtime's double-angle form and the Python
                model's fp32-angle form (runtime/vault3.c:840-849,2126-2133;
                src/vault_v3_model.py:777-794).
* ``attention`` decode attention over [sink|seg|prev|cur] with optional per-head
                seg bias (src/vault_v3_model.py:1072-1139; runtime/vault3.c:1958-2032)
                and the dense masked block-sliding prefill attention
                (src/vault_v3_model.py:805-863, 2025-2093).
* ``model``     a float64/float32 numpy restatement of the streaming step / prefill
                drivers (src/vault_v3_model.py:956-1024, 1842-2311).
* ``ref``       ctypes driver for the reference C runtime compiled from
                /root/reference/runtime/vault3.c into ``oracle/_ref`` (see Makefile).

Parity pins for every function are listed in the tests (tests/test_oracle_*.py).
"""
