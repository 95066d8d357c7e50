// rn_matrix.hpp — the host object behind rn_matrix (QuantisedMatrix): int8
// codes with per-group scales, or a codebook blob with its device tables.
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>

#include "rn_internal.hpp"

struct rn_matrix {
    int8_t* W = nullptr;
    float* sW = nullptr;
    int rows = 0, columns = 0, group = 0, form = 0;
    int bits = 0;                  // 0: int8 codes; 2, 4 or 5 (ternary): codebook indices
    unsigned char* blob = nullptr;  // codebook blob: packed indices, fp16 norms, padding
    rn::CodebookParams cb{};
    // staging of the host-slice entry points: a stream and a device buffer for
    // the input and output slices, made on first use; calls hold the mutex
    mutable std::mutex host_mu;
    mutable hipStream_t host_stream = nullptr;
    mutable char* host_buf = nullptr;
    mutable size_t host_bytes = 0;
};
