// KV-cache write (vLLM reshape_and_cache) into the paged layout read by the
// prefill and decode kernels: cache[page][slot][kv head][d] with
// page = slot_mapping[t] / page_size, slot = slot_mapping[t] % page_size.
//
// The reference has no such kernel; it only consumes this layout
// (tilelang_fa_v100/_kernels_paged.py:198-199, vLLM's cache format).
//
// One lane moves one 16-byte chunk of K and the same chunk of V, so a
// token's rows are read and written as whole 16-byte vectors (D/8 lanes per
// head row).  Tokens with a negative slot (padding) or a slot beyond the
// cache are skipped.  Purely bandwidth-bound: 2 x 2 x D bytes per (token,
// KV head) read and written.
#include "fa_common.h"
#include "fa_internal.h"

namespace fa {

__global__ __launch_bounds__(256) void cache_write_kernel(fa_cache_write_args a,
                                                          int64_t nchunks,
                                                          int64_t max_slot) {
  const int cpr = a.head_dim / 8;  // 16-byte chunks per head row
  const int cpt = a.num_kv_heads * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nchunks;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / cpt;
    const int rem = (int)(i - t * cpt);
    const int h = rem / cpr;
    const int c = rem - h * cpr;
    const int64_t slot = a.slot_mapping[t];
    if (slot < 0 || slot >= max_slot) continue;
    const int64_t page = slot / a.page_size;
    const int64_t off = slot - page * a.page_size;
    const uint16_t* ks = static_cast<const uint16_t*>(a.key) + t * a.key_stride[0] +
                         h * a.key_stride[1] + 8 * c;
    const uint16_t* vs = static_cast<const uint16_t*>(a.value) + t * a.value_stride[0] +
                         h * a.value_stride[1] + 8 * c;
    uint16_t* kd = static_cast<uint16_t*>(a.k_cache) + page * a.k_stride[0] +
                   off * a.k_stride[1] + h * a.k_stride[2] + 8 * c;
    uint16_t* vd = static_cast<uint16_t*>(a.v_cache) + page * a.v_stride[0] +
                   off * a.v_stride[1] + h * a.v_stride[2] + 8 * c;
    const u32x4 kv = ld16(ks), vv = ld16(vs);
    st16(kd, kv);
    st16(vd, vv);
  }
}

hipError_t launch_cache_write(const fa_cache_write_args& a, hipStream_t st) {
  const int64_t nchunks = (int64_t)a.num_tokens * a.num_kv_heads * (a.head_dim / 8);
  const int64_t max_slot = (int64_t)a.num_pages * a.page_size;
  // Enough workgroups to fill the chip several times; the kernel strides.
  const int64_t want = (nchunks + 255) / 256;
  const unsigned grid = (unsigned)(want < 4096 ? (want > 0 ? want : 1) : 4096);
  hipLaunchKernelGGL(cache_write_kernel, dim3(grid), dim3(256), 0, st, a, nchunks, max_slot);
  return hipGetLastError();
}

}  // namespace fa
