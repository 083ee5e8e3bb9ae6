"""Token-byte rules of the VAULT v3 decode driver (TEST INFRASTRUCTURE ONLY).

* ``tier``: segment-break tier of a token's bytes, restating runtime/vault3.c:937-959 and
  src/vault_v3_model.py:116-143 (tier 1: a newline anywhere, or a final '.', '!', '?', ';' once
  trailing ' ', TAB, CR, VT, FF are dropped; tier 2: '}', ']', '|', TAB or the pair '",'; tier 3:
  ',' or '&'; otherwise 0).
* ``system_role``: the token spells b"system" or b"system\\n" (runtime/vault3.c:1920-1928).
"""
from __future__ import annotations

import re

_T2 = re.compile(rb'[}\]|\t]|",')
_T3 = re.compile(rb"[,&]")


def tier(b: bytes) -> int:
    if not b:
        return 0
    if b"\n" in b:
        return 1
    core = re.sub(rb"[ \t\r\x0b\x0c]+$", b"", b)
    if core[-1:] in (b".", b"!", b"?", b";"):
        return 1
    if _T2.search(b):
        return 2
    if _T3.search(b):
        return 3
    return 0


def system_role(b: bytes) -> bool:
    return b in (b"system", b"system\n")
