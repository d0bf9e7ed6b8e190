// SPDX-License-Identifier: Apache-2.0
// primitives.hpp -- device prefix sums and a stable radix sort, hand-written
// for the IVF work tables and the k-means grouping (small, per-search or
// per-iteration helpers; the scans of the search itself live in kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mflat_amd {

// Prefix sum of n ints (n >= 0; the total must fit an int). Exclusive: out[i]
// = in[0] + .. + in[i - 1]; inclusive: + in[i]. out may alias in. temp holds
// scan_temp_bytes(n) bytes.
size_t scan_temp_bytes(int64_t n);
void launch_scan_i32(const int* in, int* out, int64_t n, bool inclusive, void* temp, hipStream_t s);

// Stable sort of n (key, value) pairs by the low `bits` bits of the keys
// (0 <= key < 2^bits, 1 <= bits <= 31): least-significant-digit radix sort
// on 4-bit digits; equal keys keep their input order. Outputs must not alias
// the inputs; temp holds radix_sort_temp_bytes(n, bits) bytes.
size_t radix_sort_temp_bytes(int n, int bits);
void launch_radix_sort_pairs(const int* keys_in, int* keys_out, const int* vals_in, int* vals_out, int n, int bits,
                             void* temp, hipStream_t s);

}  // namespace mflat_amd
