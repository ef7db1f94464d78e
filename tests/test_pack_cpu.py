"""Sequence packing (host): the reference's own test, the oracle, invariants."""
import numpy as np
import pytest


def test_reference_golden_vector():
    from ceo_amd.data import pack_sequences

    # dataset.zig:467-481
    p = pack_sequences([[1, 2, 3], [4, 5], [6, 7, 8, 9]], 20)
    assert p.tokens.size == 9 and p.num_sequences == 3
    assert p.tokens.tolist() == [1, 2, 3, 4, 5, 6, 7, 8, 9]
    assert p.positions.tolist() == [0, 1, 2, 0, 1, 0, 1, 2, 3]
    assert p.sequence_ids.tolist() == [0, 0, 0, 1, 1, 2, 2, 2, 2]
    assert p.cumulative_lengths.tolist() == [3, 5, 9]
    assert p.cu_seqlens.tolist() == [0, 3, 5, 9] and p.cu_seqlens.dtype == np.int32


def test_sequences_that_do_not_fit_are_skipped():
    from ceo_amd.data import pack_sequences

    p = pack_sequences([[1, 2, 3], [4, 5, 6, 7, 8], [9], [10, 11]], 6)
    assert p.tokens.tolist() == [1, 2, 3, 9, 10, 11]
    assert p.cu_seqlens.tolist() == [0, 3, 4, 6]
    assert p.sequence_ids.tolist() == [0, 0, 0, 1, 2, 2]


@pytest.mark.parametrize("seed", range(6))
def test_matches_oracle(oracle, seed):
    from ceo_amd.data import pack_sequences

    rng = np.random.default_rng(seed)
    seqs = [rng.integers(0, 50000, rng.integers(0, 300)) for _ in range(rng.integers(0, 40))]
    cap = int(rng.integers(1, 4000))
    p = pack_sequences(seqs, cap)
    toks, pos, sid, cum = oracle.pack_sequences([s.tolist() for s in seqs], cap)
    assert p.tokens.tolist() == toks and p.positions.tolist() == pos
    assert p.sequence_ids.tolist() == sid and p.cumulative_lengths.tolist() == cum
    assert p.num_sequences == len(cum) and p.cu_seqlens[0] == 0
    assert np.all(np.diff(p.cu_seqlens) >= 0) and p.cu_seqlens[-1] <= cap


def test_empty_input_and_errors():
    import ctypes

    from ceo_amd._lib import lib
    from ceo_amd.data import pack_sequences

    p = pack_sequences([], 10)
    assert p.num_sequences == 0 and p.tokens.size == 0 and p.cu_seqlens.tolist() == [0]
    n = ctypes.c_size_t()
    assert lib().efla_pack_sequences(None, None, 1, 10, None, None, None, None,
                                     ctypes.byref(n), ctypes.byref(n)) == 1
    assert lib().efla_pack_sequences(None, None, 0, 1 << 40, None, None, None, None,
                                     ctypes.byref(n), ctypes.byref(n)) == 9


def test_chunked_scan_ranges_reference_test():
    from ceo_amd.state import ChunkedScan

    # efla.zig:497-505
    s = ChunkedScan(10000, 1024)
    assert s.chunk_size == 1024 and s.num_chunks == 10
    assert s.get_chunk_range(5) == (5120, 6144)
    # the reference clips to num_chunks * chunk_size (10240), not to 10000
    assert s.get_chunk_range(9) == (9216, 10240)
