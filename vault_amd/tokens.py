"""Token byte strings of a VLT3 file (the VTOK blob) and the per-token rules the decode driver reads
from them.

VTOK layout (tools/vlt3.py:246-305; validated by runtime/vault3.c:427-453): a 128-byte head
``"VTOK", version 1, n_vocab, n_merges, n_special, n_ranges, 0`` followed by six little-endian u64
section offsets (table, pool, merges, specials, ranges, byte map).  The table holds one
``(pool offset u32, length u32)`` pair per token; the byte map holds, for each of the 256 raw
bytes, the id of the token that spells that byte.  Merges, specials and ranges belong to the
tokenizer (not part of this path) and are carried through unread.

Rules derived from the token bytes:

* ``break_tier``: segment-break tier of a token (runtime/vault3.c:937-959;
  src/vault_v3_model.py:116-143): 1 when the bytes hold a newline or end (ignoring trailing ASCII
  white space) in one of ``. ! ? ;``; else 2 for ``} ] | TAB`` or a ``",`` pair; else 3 for ``,`` or
  ``&``; else 0.  Empty strings are tier 0.
* ``is_system_role``: the token spells ``system`` or ``system\\n`` (runtime/vault3.c:1920-1928).
* ``newline_id``: the byte map's token for ``\\n`` (runtime/vault3.c:2047).

Without a token table (a model built from tensors alone, like the reference Python model offline)
the driver uses the Python reference's rules instead: every tier 0, ``system_tok_id`` from the
config, newline id 198 (src/vault_v3_model.py:2224-2252).
"""
from __future__ import annotations

import struct
from typing import List, Optional, Sequence

import numpy as np

HEAD = 128
_HEAD = struct.Struct("<4sIIIIII6Q")
_TRAIL_WS = b" \t\r\x0b\x0c"


class VTOKError(ValueError):
    pass


def break_tier(b: bytes) -> int:
    """Segment-break tier of one token's bytes (runtime/vault3.c:937-959)."""
    if not b:
        return 0
    t2 = t3 = False
    n = len(b)
    for i, ch in enumerate(b):
        if ch == 0x0A:
            return 1
        if ch in (0x7D, 0x5D, 0x7C, 0x09):
            t2 = True
        elif ch == 0x22 and i + 1 < n and b[i + 1] == 0x2C:
            t2 = True
        elif ch in (0x2C, 0x26):
            t3 = True
    core = b.rstrip(_TRAIL_WS)
    if core and core[-1] in (0x2E, 0x21, 0x3F, 0x3B):
        return 1
    return 2 if t2 else (3 if t3 else 0)


class TokenTable:
    """Token strings of one model: ``bytes_of(id)``, the break-tier table, system-role test and
    newline id.  Ids at or beyond ``n_vocab`` have no bytes (runtime/vault3.c:2303-2308)."""

    def __init__(self, token_bytes: Sequence[bytes], byte_map: Sequence[int], vocab_size: int):
        self.tokens: List[bytes] = [bytes(t) for t in token_bytes]
        self.byte_map = np.asarray(byte_map, dtype=np.int64)
        if self.byte_map.shape != (256,):
            raise VTOKError("byte map must have 256 entries")
        self.n_vocab = len(self.tokens)
        self.vocab_size = int(vocab_size)
        tiers = np.zeros(self.vocab_size, dtype=np.uint8)
        for i, t in enumerate(self.tokens[:self.vocab_size]):
            if t:
                tiers[i] = break_tier(t)
        self.tiers = tiers

    def bytes_of(self, tid: int) -> bytes:
        return self.tokens[tid] if 0 <= tid < self.n_vocab else b""

    def is_system_role(self, tid: int) -> bool:
        b = self.bytes_of(tid)
        return b == b"system" or b == b"system\n"

    @property
    def newline_id(self) -> int:
        return int(self.byte_map[0x0A])

    @property
    def has_strings(self) -> bool:
        return any(self.tokens)

    # ------------------------------------------------------------------ VTOK blob
    @classmethod
    def from_vtok(cls, blob: bytes, vocab_size: int) -> "TokenTable":
        """Parse and validate a VTOK blob with the checks of runtime/vault3.c:427-453."""
        if len(blob) < HEAD:
            raise VTOKError("VTOK blob shorter than its head")
        magic, ver, n_vocab, n_merges, n_special, n_ranges, _, o_tab, o_pool, o_mer, o_spc, o_rng, o_byt = \
            _HEAD.unpack_from(blob, 0)
        if magic != b"VTOK" or ver != 1:
            raise VTOKError("bad VTOK magic / version")
        if n_vocab == 0 or n_vocab > vocab_size or n_merges > 2097152 or n_special > n_vocab or n_ranges > 65536:
            raise VTOKError("VTOK counts out of range")
        size = len(blob)

        def region(o, n):
            return o % 4 == 0 and o <= size and n <= size - o

        s_tab, s_mer, s_spc, s_rng, s_byt = 8 * n_vocab, 12 * n_merges, 4 * n_special, 12 * n_ranges, 1024
        if not (region(o_tab, s_tab) and region(o_mer, s_mer) and region(o_spc, s_spc) and region(o_rng, s_rng)
                and region(o_byt, s_byt)) or o_pool > o_mer or o_pool < o_tab + s_tab:
            raise VTOKError("VTOK section out of bounds")
        pool_size = o_mer - o_pool
        tab = np.frombuffer(blob, dtype="<u4", count=2 * n_vocab, offset=o_tab).reshape(n_vocab, 2).astype(np.int64)
        if np.any(tab[:, 0] > pool_size) or np.any(tab[:, 1] > pool_size - tab[:, 0]):
            raise VTOKError("token string outside the pool")
        if n_merges:
            mer = np.frombuffer(blob, dtype="<u4", count=3 * n_merges, offset=o_mer)
            if np.any(mer >= n_vocab):
                raise VTOKError("merge id out of range")
        if n_special and np.any(np.frombuffer(blob, dtype="<u4", count=n_special, offset=o_spc) >= n_vocab):
            raise VTOKError("special id out of range")
        byte_map = np.frombuffer(blob, dtype="<u4", count=256, offset=o_byt).astype(np.int64)
        if np.any(byte_map >= n_vocab):
            raise VTOKError("byte map id out of range")
        pool = blob[o_pool:o_mer]
        toks = [pool[o:o + n] for o, n in tab.tolist()]
        return cls(toks, byte_map, vocab_size)

    def to_vtok(self) -> bytes:
        return build_vtok(self.tokens, self.byte_map.tolist())


def build_vtok(token_bytes: Sequence[bytes], byte_map: Optional[Sequence[int]] = None) -> bytes:
    """A VTOK blob holding these token strings (no merges, specials or ranges); ``byte_map`` defaults
    to token 0 for every byte.  Sections are 8-byte aligned as in tools/vlt3.py:283-299."""
    n = len(token_bytes)
    if n == 0:
        raise VTOKError("empty vocabulary")
    bm = [0] * 256 if byte_map is None else [int(x) for x in byte_map]
    pool = bytearray()
    tab = np.zeros((n, 2), dtype="<u4")
    for i, t in enumerate(token_bytes):
        tab[i] = (len(pool), len(t))
        pool += t
    sections = [tab.tobytes(), bytes(pool), b"", b"", b"", np.asarray(bm, dtype="<u4").tobytes()]
    offs, cur = [], HEAD
    for s in sections:
        cur = (cur + 7) & ~7
        offs.append(cur)
        cur += len(s)
    blob = bytearray(_HEAD.pack(b"VTOK", 1, n, 0, 0, 0, 0, *offs).ljust(HEAD, b"\0"))
    for o, s in zip(offs, sections):
        blob += b"\0" * (o - len(blob))
        blob += s
    return bytes(blob)
