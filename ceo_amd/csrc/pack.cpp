// Host-side sequence packing: the data format on the caller's side of the
// varlen EFLA entries.  Replaces packSequences (src/data/dataset.zig:421-465)
// and adds the int32 cu_seqlens array (leading 0) that efla_chunk_*_hip take,
// where the reference's PackedSequence.cumulative_lengths has no leading 0.
//
// Greedy, in input order: a sequence that does not fit in what is left of
// max_length is skipped and packing goes on with the next one (dataset.zig:
// 442-446).  For each packed token: its id, its position within its sequence
// and the index of its sequence among the packed ones.
#include <stddef.h>
#include <stdint.h>

#include "../../include/efla_hip.h"

extern "C" int efla_pack_sequences(const uint32_t* tokens, const size_t* lengths,
                                   size_t num_sequences_in, size_t max_length,
                                   uint32_t* packed_tokens, size_t* positions,
                                   size_t* sequence_ids, int32_t* cu_seqlens,
                                   size_t* num_tokens_out, size_t* num_sequences_out) {
    if (!num_tokens_out || !num_sequences_out) return 1;
    if (num_sequences_in != 0 && (!tokens || !lengths)) return 1;
    if (max_length > (size_t)INT32_MAX) return 9;  // cu_seqlens is int32
    size_t len = 0, seq = 0, src = 0;
    if (cu_seqlens) cu_seqlens[0] = 0;
    for (size_t s = 0; s < num_sequences_in; ++s) {
        const size_t n = lengths[s];
        const uint32_t* in = tokens + src;
        src += n;
        if (n > max_length - len) continue;  // does not fit: skipped
        for (size_t p = 0; p < n; ++p) {
            if (packed_tokens) packed_tokens[len + p] = in[p];
            if (positions) positions[len + p] = p;
            if (sequence_ids) sequence_ids[len + p] = seq;
        }
        len += n;
        ++seq;
        if (cu_seqlens) cu_seqlens[seq] = (int32_t)len;
    }
    *num_tokens_out = len;
    *num_sequences_out = seq;
    return 0;
}
