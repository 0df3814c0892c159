// Launchers behind the C ABI (fa_capi.cpp).  Arguments are validated by the
// caller; these only configure grids and enqueue kernels on `st`.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

#include "fa355.h"
#include "fa_tiles.h"

namespace fa {

hipError_t launch_fwd(const fa_fwd_args& a, hipStream_t st);

// bwd_workspace_bytes: the dS-store path's workspace where it applies
// (head_dim 128 or 256, causal or full attention, dS tiles below
// tiles::kBwdDsMaxBytes), else the row statistics only.
// bwd_min_workspace_bytes: the row statistics (the recompute path).
size_t bwd_workspace_bytes(const fa_bwd_args& a);
size_t bwd_min_workspace_bytes(const fa_bwd_args& a);
hipError_t launch_bwd(const fa_bwd_args& a, void* ws, size_t ws_bytes, hipStream_t st);

int paged_grid_slots(const fa_paged_args& a);
hipError_t launch_paged_prefill(const fa_paged_args& a, hipStream_t st);
// Split-KV paged prefill: nsplit in [1, kMaxPagedSplits]; ws holds
// paged_split_workspace_bytes(a, nsplit) bytes (none for nsplit == 1).
constexpr int kMaxPagedSplits = tiles::kMaxSplits;
int paged_num_splits(const fa_paged_args& a);
size_t paged_split_workspace_bytes(const fa_paged_args& a, int nsplit);
hipError_t launch_paged_prefill_split(const fa_paged_args& a, int nsplit, void* ws,
                                      hipStream_t st);

// Compute units of the current device (cached per device).
int device_cu_count();

// Grid of a persistent launch over ntiles x nbh tiles (persistent_tile in
// fa_common.h): per_cu workgroups per CU, fewer when there are fewer tiles,
// a multiple of 8 when nbh is a multiple of 8 (each workgroup then stays on
// one XCD's heads).
inline int persistent_grid(int ntiles, int nbh, int per_cu) {
  const int64_t total = (int64_t)ntiles * nbh;
  int64_t w = std::min<int64_t>(total, (int64_t)per_cu * device_cu_count());
  if (nbh % 8 == 0) w = std::max<int64_t>(8, w / 8 * 8);
  return (int)w;
}

int decode_num_splits(const fa_decode_args& a);
size_t decode_workspace_bytes(const fa_decode_args& a);
hipError_t launch_decode(const fa_decode_args& a, void* ws, hipStream_t st);

// Device address of the current device's FA_NOALLOC_SCRATCH_BYTES-byte
// static scratch array (fa_scratch.hip), looked up on the first call per
// device.
hipError_t noalloc_scratch(void** ptr);

hipError_t launch_cache_write(const fa_cache_write_args& a, hipStream_t st);

}  // namespace fa
