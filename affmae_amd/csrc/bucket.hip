// Stable bucketing of (key, payload) pairs: hipCUB radix sort, then a
// lower_bound per key for the bucket offsets (see bucket.hpp).
#include "bucket.hpp"

#include <hipcub/device/device_radix_sort.hpp>

namespace aff {
namespace bucket {

namespace {
constexpr int THREADS = 256;

// off[k] = first position of key >= k in the sorted keys, k = 0 .. nkeys.
__global__ __launch_bounds__(THREADS) void offsets_kernel(const unsigned *keys, int64_t count, int nkeys, int *off) {
    const int k = blockIdx.x * THREADS + threadIdx.x;
    if (k > nkeys) return;
    int64_t lo = 0, hi = count;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (keys[mid] < unsigned(k)) lo = mid + 1;
        else hi = mid;
    }
    off[k] = int(lo);
}
}  // namespace

int key_bits(int64_t max_key) {
    int bits = 1;
    while (bits < 32 && ((int64_t)1 << bits) <= max_key) ++bits;
    return bits;
}

size_t sort_temp_bytes(int64_t count, int bits) {
    size_t bytes = 0;
    hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, static_cast<const unsigned *>(nullptr),
                                       static_cast<unsigned *>(nullptr), static_cast<const int *>(nullptr),
                                       static_cast<int *>(nullptr), (int)count, 0, bits, (hipStream_t)0);
    return bytes;
}

aff_status sort_and_offsets(const unsigned *keys_in, const int *vals_in, unsigned *keys_out, int *vals_out,
                            int64_t count, int nkeys, void *temp, size_t temp_bytes, int *off, hipStream_t stream) {
    if (count > 0) {
        size_t tb = temp_bytes;
        if (hipcub::DeviceRadixSort::SortPairs(temp, tb, keys_in, keys_out, vals_in, vals_out, (int)count, 0,
                                               key_bits(nkeys), stream) != hipSuccess)
            return fail(AFF_ERR_LAUNCH, "bucket sort: radix sort of %lld pairs failed", (long long)count);
    }
    hipLaunchKernelGGL(offsets_kernel, dim3((unsigned)((nkeys + 1 + THREADS - 1) / THREADS)), dim3(THREADS), 0, stream,
                       keys_out, count, nkeys, off);
    return check_launch("bucket sort (offsets)");
}

}  // namespace bucket
}  // namespace aff
