// Sequence / chunk bookkeeping shared by the chunked EFLA kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace efla {
namespace q {

constexpr int BT = 64;  // chunk length

// Where the tokens of each sequence live.  Without cu_seqlens there are N
// sequences of T tokens back to back; with it, `cu` is a sanitised copy of
// cu_seqlens and `coff[i]` the index of sequence i's first chunk.  `order`
// (varlen, at most LPT_MAX_SEQS sequences; else NULL) lists the sequences by
// decreasing chunk count, ties in index order: the scans, one chain of
// dependent chunks per workgroup, take the longest sequences first so that no
// long chain starts late.
struct SeqInfo {
    const int32_t* cu;
    const int32_t* coff;
    const int32_t* order;
    int N;
    long T;
    int nt;  // chunks per sequence (fixed-length case)
};

constexpr int LPT_MAX_SEQS = 1024;  // one sequence per thread of the offsets kernel

// The scans' (sequence * H + head) index of workgroup id's row, longest
// sequences first where `order` is given.
__device__ __forceinline__ int scan_seq_head(const SeqInfo& s, int bh, int H) {
    return s.order ? s.order[bh / H] * H + bh % H : bh;
}

__device__ __forceinline__ void seq_bounds(const SeqInfo& s, int seq, long& bos, long& len,
                                           int& slot0) {
    if (s.cu == nullptr) {
        bos = (long)seq * s.T;
        len = s.T;
        slot0 = seq * s.nt;
    } else {
        bos = s.cu[seq];
        len = (long)s.cu[seq + 1] - bos;
        slot0 = s.coff[seq];
    }
}

// Elements between consecutive tokens of the head-sliced q, k, v inputs and
// dq, dk, dv outputs of the bf16 kernels: H*K, H*K, H*V for packed
// (tokens, H, D) arrays, more when each is a column slice of a wider row
// (a fused projection).  grad_output, output and beta stay packed.
struct TokLd {
    long q, k, v, dq, dk, dv;
};

// Chunk slot -> first token and length; false for slots past the last chunk.
__device__ __forceinline__ bool locate_chunk(const SeqInfo& s, int slot, long& bos, int& len) {
    if (s.cu == nullptr) {
        const int seq = slot / s.nt, n = slot - seq * s.nt;
        if (seq >= s.N) return false;
        bos = (long)seq * s.T + (long)n * BT;
        const long rem = s.T - (long)n * BT;
        len = (int)(rem < BT ? rem : BT);
        return true;
    }
    if (slot >= s.coff[s.N]) return false;
    int lo = 0, hi = s.N - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s.coff[mid] <= slot) lo = mid;
        else hi = mid - 1;
    }
    const int n = slot - s.coff[lo];
    bos = (long)s.cu[lo] + (long)n * BT;
    const long rem = (long)s.cu[lo + 1] - bos;
    len = (int)(rem < BT ? rem : BT);
    return true;
}

}  // namespace q
}  // namespace efla
