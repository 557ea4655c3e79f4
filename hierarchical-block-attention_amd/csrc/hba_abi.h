// Host-side argument checks and dtype/head-dim dispatch shared by the entry points.
#pragma once

#include <stdint.h>

#include "../../include/hba_amd.h"

namespace hba {
namespace abi {

inline int check_dtype_dim(int dtype, int64_t d) {
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    if (d != 64 && d != 128) return HBA_ERR_UNSUPPORTED;
    return HBA_OK;
}

inline bool aligned16(const void *p) { return (((uintptr_t)p) & 15u) == 0; }

inline int64_t elem_size(int dtype) { return dtype == HBA_DTYPE_BF16 ? 2 : 4; }

// Rows of a [B, n, H, d] view start on 16-byte boundaries.
inline bool rows_aligned(int dtype, const void *p, const int64_t s[3]) {
    int64_t q = 16 / elem_size(dtype);
    return aligned16(p) && s[0] % q == 0 && s[1] % q == 0 && s[2] % q == 0;
}

}  // namespace abi
}  // namespace hba

#define HBA_DISPATCH_DT_D(dtype, d, M)          \
    do {                                        \
        if ((dtype) == HBA_DTYPE_F32) {         \
            if ((d) == 64) M(0, 64);            \
            else M(0, 128);                     \
        } else {                                \
            if ((d) == 64) M(1, 64);            \
            else M(1, 128);                     \
        }                                       \
    } while (0)
