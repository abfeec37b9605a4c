// The library's own stable LSD radix sort (radix.hip), for the other kernel
// files: keys of 32 or 64 bits, optionally with int32 values.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace spira_hip {

// Workspace bytes of sort_keys_values for n keys (with_values: vals_out is
// given).
template <typename CT> size_t sort_bytes(int64_t n, bool with_values);

// Stable ascending sort of keys_in into keys_out; with vals_out, the values
// follow their keys (vals_in null: the values are the input indices
// 0 .. n - 1).  The inputs are left unchanged; n < 2^30.
template <typename CT>
int sort_keys_values(const CT *keys_in, const int32_t *vals_in, CT *keys_out, int32_t *vals_out, int64_t n,
                     void *ws, size_t ws_bytes, hipStream_t s);

// Waits for `s` and reports whether the last sort that used `ws` had a
// look-back wait run out (its output is then incomplete).
template <typename CT> int sort_status(const void *ws, int64_t n, bool with_values, hipStream_t s);

}  // namespace spira_hip
