// qr_host.h -- host-only helpers of the C-ABI (qr_host.cpp).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "qr_formats.h"

namespace qr {

// Whether every page of the host range [p, p + bytes) is readable (and, when
// `write`, writable) by this process; probed without raising a signal.
bool host_range_ok(const void* p, size_t bytes, bool write);

// Formats m4_bridge_dispatch_gemm accepts, and every format with kernels.
bool is_projection_format(int f);
bool has_kernels(int f);

// Argument validation of a projection: 0, or the reference's codes -2 / -3 /
// -4 in its order (core/bridge/m4_mlx_bridge.mm:204-230, minus the init
// check); `ext` widens the format range to every format with kernels.
int validate(const void* X, size_t Xb, const void* W, size_t Wb, const void* Y, size_t Yb, int format,
             uint32_t M, uint32_t K, uint32_t N, bool ext = false);

}  // namespace qr
