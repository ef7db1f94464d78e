"""EFLA state carry across segments: transitions, the affine combine, and the
sequence-sharded forward it enables.

Mirrors the reference's ``EflaState`` (src/model/efla.zig:13-86: a
(heads, d_k, d_v) state carried between calls) and ``ChunkedScan``
(efla.zig:454-485, whose ``prefixScan`` is empty and whose CUDA counterpart
``efla_chunked_scan_cuda`` sums states, efla.cu:711-748).  The combine the
recurrence needs is affine: over a segment, S_out = A S_in + B with
A = prod_t (I - c_t k_t k_t^T) and B the segment's final state from zero.

``sharded_forward`` is the sequence-parallel forward of a multi-GPU design run
on one device: split every sequence into P segments, run each segment from a
zero state (keeping its final state B_p) and its transition A_p, combine with
``efla_affine_state_scan_hip``, then run each segment again from its true
incoming state.  On P devices the first and last passes are local and only the
(A_p, B_p) exchange crosses devices.
"""
from __future__ import annotations

import ctypes

import torch

from . import efla
from ._lib import check, lib


class ChunkedScan:
    """Chunk ranges over a sequence (efla.zig:454-471), with the affine
    prefix combine in place of the reference's empty ``prefixScan``."""

    def __init__(self, seq_len: int, chunk_size: int):
        self.chunk_size = chunk_size
        self.num_chunks = (seq_len + chunk_size - 1) // chunk_size

    def get_chunk_range(self, idx: int):
        """(start, end) as efla.zig:465-470 computes them: the end is clipped
        to num_chunks * chunk_size, not to the sequence length."""
        start = idx * self.chunk_size
        return start, min(start + self.chunk_size, self.num_chunks * self.chunk_size)

    @staticmethod
    def prefix_scan(transitions, states) -> None:
        """states[i] = transitions[i] @ states[i-1] + states[i] in place."""
        affine_state_scan(transitions, states)


def affine_state_scan(transitions, states) -> None:
    """In-place affine combine over segment states (lists of fp32 device
    tensors (N, H, d_k, d_v) and transitions (N, H, d_k, d_k))."""
    n = len(states)
    if n == 0:
        return
    N, H, K, V = states[0].shape
    for s in states:
        efla._require(s, "state", torch.float32)
    for a in transitions[1:]:
        efla._require(a, "transition", torch.float32)
        if tuple(a.shape) != (N, H, K, K):
            raise ValueError("transition must be (N, H, d_k, d_k)")
    vp = ctypes.c_void_p
    tr = (vp * n)(*([None] + [a.data_ptr() for a in transitions[1:]]))
    st = (vp * n)(*[s.data_ptr() for s in states])
    rc = lib().efla_affine_state_scan_hip(tr, st, n, N * H, K, V, efla._stream(states[0]))
    check(rc, "efla_affine_state_scan_hip")


def chunk_transition(q, k, beta, cu_seqlens=None) -> torch.Tensor:
    """A = prod_t (I - c_t k_t k_t^T) per (sequence, head), fp32 (N, H, K, K):
    the chunked forward's final state from S_0 = I with v = 0."""
    B, T, H, K = k.shape
    N = B if cu_seqlens is None else cu_seqlens.numel() - 1
    eye = torch.eye(K, dtype=torch.float32, device=k.device).expand(N, H, K, K).contiguous()
    zeros = torch.zeros(B, T, H, K, dtype=k.dtype, device=k.device)
    _, A = efla.chunk_efla_fwd(q, k, zeros, beta, initial_state=eye, output_final_state=True,
                               cu_seqlens=cu_seqlens)
    return A


def sharded_forward(q, k, v, beta, segments: int, initial_state=None):
    """Chunked EFLA forward of (B, T, H, *) inputs with every sequence split
    into `segments` consecutive pieces (T divisible by 64 * segments), combined
    through the affine state scan.  Returns (o, final_state) as chunk_efla_fwd
    with output_final_state=True would."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if T % (64 * segments) != 0:
        raise ValueError("T must split into whole 64-token chunks per segment")
    L = T // segments
    parts = [slice(p * L, (p + 1) * L) for p in range(segments)]
    seg = [{n: t[:, s].contiguous() for n, t in (("q", q), ("k", k), ("v", v),
                                                  ("beta", beta))} for s in parts]
    # pass 1 (local per device): B_p from a zero start (the first segment from
    # the caller's initial state), A_p for the others
    states, trans = [], [None]
    for p, x in enumerate(seg):
        s0 = initial_state if p == 0 else None
        _, st = efla.chunk_efla_fwd(x["q"], x["k"], x["v"], x["beta"], initial_state=s0,
                                    output_final_state=True)
        states.append(st)
        if p > 0:
            trans.append(chunk_transition(x["q"], x["k"], x["beta"]))
    # the exchange: S_p = A_p S_{p-1} + B_p
    affine_state_scan(trans, states)
    # pass 2 (local): each segment from its true incoming state
    outs = []
    for p, x in enumerate(seg):
        s_in = initial_state if p == 0 else states[p - 1]
        o, _ = efla.chunk_efla_fwd(x["q"], x["k"], x["v"], x["beta"], initial_state=s_in)
        outs.append(o)
    return torch.cat(outs, dim=1), states[-1]
