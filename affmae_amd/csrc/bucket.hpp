// Stable bucketing of (key, payload) pairs, shared by the backward passes.
//
// The backward kernels turn scattered sums (every pair adds into the row its
// key names) into gathers: the pairs are sorted by key with a stable radix
// sort, so each bucket lists its pairs in payload order, and off[k] is the
// first position whose key is >= k.  A bucket is then summed in that order,
// which makes the result independent of scheduling.
#pragma once

#include "common.hpp"

namespace aff {
namespace bucket {

// Smallest bit count that holds every key in [0, max_key].
int key_bits(int64_t max_key);

// Bytes of radix-sort scratch for `count` pairs with `bits`-bit keys.
size_t sort_temp_bytes(int64_t count, int bits);

// Sorts (keys_in, vals_in) by key (stable) into (keys_out, vals_out) using
// `temp` (sort_temp_bytes bytes) and writes off[0 .. nkeys].  Keys must lie in
// [0, nkeys]; key nkeys marks pairs that belong to no bucket (they sort last).
aff_status sort_and_offsets(const unsigned *keys_in, const int *vals_in, unsigned *keys_out, int *vals_out,
                            int64_t count, int nkeys, void *temp, size_t temp_bytes, int *off, hipStream_t stream);

}  // namespace bucket
}  // namespace aff
