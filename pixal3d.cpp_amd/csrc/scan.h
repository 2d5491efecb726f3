// Device-wide exclusive prefix sum used by the topology kernels.
#pragma once

#include "pxs_common.h"

namespace pxs {

// Elements reduced per scan block (256 threads x 8 items).
constexpr int kScanBlock = 256;
constexpr int kScanItems = 8;
constexpr int64_t kScanTile = static_cast<int64_t>(kScanBlock) * kScanItems;

// Scratch bytes the scan needs for `count` items (block partials + total).
size_t scan_workspace_bytes(int64_t count);

// out[i] = sum_{j<i} value(i) for i < count, and *total = sum of all, where
// value(i) = in[i] (int32 input) or popcount(in[i]) when popcount is set.
// out may alias nothing; total is a device int64.  Up to 16384 items: one
// single-workgroup launch.  Above that, three launches:
// per-tile sums, a single-block scan of the tile sums, per-tile scans.
int exclusive_scan_i32(const int32_t * in, int64_t * out, int64_t count, int64_t * total,
                       void * workspace, hipStream_t stream);
int exclusive_scan_popcount(const uint32_t * in, int64_t * out, int64_t count, int64_t * total,
                            void * workspace, hipStream_t stream);

// Fill helpers (kernels, not hipMemsetAsync, so the calls stay capturable).
int fill_i32(int32_t * p, int64_t count, int32_t value, hipStream_t stream);
int fill_i64(int64_t * p, int64_t count, int64_t value, hipStream_t stream);
int fill_u32(uint32_t * p, int64_t count, uint32_t value, hipStream_t stream);

} // namespace pxs
