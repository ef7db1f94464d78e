"""Sequence packing for the varlen EFLA entries (host side, no GPU).

Mirrors ``packSequences`` / ``PackedSequence`` (src/data/dataset.zig:404-465)
over the library's ``efla_pack_sequences``, and adds ``cu_seqlens``: the
int32 offsets with a leading 0 that ``chunk_efla_fwd`` / ``chunk_efla_bwd``
take (the reference's ``cumulative_lengths`` are ``cu_seqlens[1:]``).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib


@dataclass
class PackedSequence:
    tokens: np.ndarray               # uint32, packed token ids
    positions: np.ndarray            # uint64, index within its sequence
    sequence_ids: np.ndarray         # uint64, index of its sequence among the packed
    cumulative_lengths: np.ndarray   # uint64, end offset of each packed sequence
    cu_seqlens: np.ndarray           # int32, (num_sequences + 1,), leading 0
    num_sequences: int

    def cu_seqlens_device(self, device="cuda"):
        import torch

        return torch.from_numpy(self.cu_seqlens).to(device)


def pack_sequences(sequences, max_length: int) -> PackedSequence:
    """Greedy packing in order; a sequence that does not fit is skipped."""
    seqs = [np.ascontiguousarray(s, dtype=np.uint32).ravel() for s in sequences]
    lengths = np.array([s.size for s in seqs], dtype=np.uint64)
    flat = np.concatenate(seqs) if seqs else np.zeros(0, np.uint32)
    cap = max(int(max_length), 1)
    toks = np.empty(cap, np.uint32)
    pos = np.empty(cap, np.uint64)
    sid = np.empty(cap, np.uint64)
    cu = np.empty(len(seqs) + 1, np.int32)
    nt, ns = ctypes.c_size_t(), ctypes.c_size_t()
    vp = ctypes.c_void_p
    rc = lib().efla_pack_sequences(vp(flat.ctypes.data) if flat.size else vp(0),
                                   vp(lengths.ctypes.data) if lengths.size else vp(0),
                                   len(seqs), int(max_length), vp(toks.ctypes.data),
                                   vp(pos.ctypes.data), vp(sid.ctypes.data),
                                   vp(cu.ctypes.data), ctypes.byref(nt), ctypes.byref(ns))
    check(rc, "efla_pack_sequences")
    n, s = nt.value, ns.value
    return PackedSequence(toks[:n].copy(), pos[:n].copy(), sid[:n].copy(),
                          cu[1:s + 1].astype(np.uint64), cu[:s + 1].copy(), s)
