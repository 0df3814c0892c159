// extern "C" entry points of libfa355.so (declared in include/fa355.h).
//
// Every entry point validates its arguments completely before enqueueing any
// work, so a rejected call has no device-side effect.  No entry point
// allocates, frees or synchronises; all run asynchronously on the caller's
// stream.  The reference exposes the same operations as TileLang JIT kernels
// invoked from Python (tilelang_fa_v100/interface.py:35-36,52;
// _paged_adapter.py:40-46; _decode_adapter.py:46).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <cstdarg>
#include <cstring>

#include "fa355.h"
#include "fa_internal.h"

namespace {

thread_local char g_msg[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_msg[0] = '\0';
  return FA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(FA_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool strides_ok(const int64_t* s, int n) {
  for (int i = 0; i < n; ++i)
    if (s[i] < 0 || (s[i] & 7) != 0) return false;
  return true;
}

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

constexpr int64_t kIntMax = 0x7fffffff;

// Kernels address up to 32 rows past a uniform row base with unsigned 32-bit
// offsets, so per-row (sequence) strides must stay below 2^26 elements.
constexpr int64_t kMaxRowStride = int64_t(1) << 26;
constexpr int64_t kMaxFwdKvRowStride = int64_t(1) << 24;

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA355_ABI_VERSION; }

const char* fa_last_error_message(void) { return g_msg; }

const char* fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "success";
    case FA_E_INVALID: return "invalid argument";
    case FA_E_UNSUPPORTED: return "unsupported configuration";
    case FA_E_HIP: return "HIP runtime error";
    case FA_E_WORKSPACE: return "workspace missing or too small";
  }
  return "unknown status";
}

// ------------------------------------------------------------------ dense fwd

static int check_fwd(const fa_fwd_args* a) {
  if (!a) return fail(FA_E_INVALID, "fa_fwd: null args");
  if (!a->q || !a->k || !a->v || !a->out)
    return fail(FA_E_INVALID, "fa_fwd: null tensor pointer");
  if (a->dtype != FA_DTYPE_F16 && a->dtype != FA_DTYPE_BF16)
    return fail(FA_E_UNSUPPORTED, "fa_fwd: dtype %d not supported", a->dtype);
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(FA_E_UNSUPPORTED, "fa_fwd: head_dim %d not in {64,128,256}", a->head_dim);
  if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_k < 0)
    return fail(FA_E_INVALID, "fa_fwd: negative size");
  if (a->num_heads <= 0 || a->num_heads_k <= 0 || a->num_heads % a->num_heads_k != 0)
    return fail(FA_E_INVALID, "fa_fwd: num_heads %d not a multiple of num_heads_k %d",
                a->num_heads, a->num_heads_k);
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out))
    return fail(FA_E_UNSUPPORTED, "fa_fwd: tensors must be 16-byte aligned");
  if (!strides_ok(a->q_stride, 3) || !strides_ok(a->k_stride, 3) ||
      !strides_ok(a->v_stride, 3) || !strides_ok(a->o_stride, 3))
    return fail(FA_E_UNSUPPORTED, "fa_fwd: strides must be non-negative multiples of 8");
  if (a->has_window && (a->window_left < -1 || a->window_right < -1))
    return fail(FA_E_INVALID, "fa_fwd: window sizes must be >= -1");
  // The head_dim 128 core DMAs K / V tiles through buffer resources with
  // 32-bit lane offsets of up to 64 rows.
  if (a->k_stride[1] >= kMaxFwdKvRowStride || a->v_stride[1] >= kMaxFwdKvRowStride)
    return fail(FA_E_UNSUPPORTED, "fa_fwd: k / v sequence strides must be below 2^24 elements");
  const int64_t tiles = ((int64_t)a->seqlen_q + 127) / 128 * a->num_heads * a->batch;
  if (tiles > kIntMax) return fail(FA_E_UNSUPPORTED, "fa_fwd: problem too large");
  return ok();
}

int fa_fwd(const fa_fwd_args* a, void* stream) {
  const int st = check_fwd(a);
  if (st != FA_OK) return st;
  // seqlen_k == 0 still launches: every row is written as out = 0, lse = -inf.
  if (a->batch == 0 || a->seqlen_q == 0) return ok();
  return hip_status(fa::launch_fwd(*a, static_cast<hipStream_t>(stream)), "fa_fwd launch");
}

// ------------------------------------------------------------------ dense bwd

static int check_bwd(const fa_bwd_args* a) {
  if (!a) return fail(FA_E_INVALID, "fa_bwd: null args");
  if (!a->q || !a->k || !a->v || !a->out || !a->dout || !a->lse || !a->dq || !a->dk ||
      !a->dv)
    return fail(FA_E_INVALID, "fa_bwd: null tensor pointer");
  if (a->dtype != FA_DTYPE_F16 && a->dtype != FA_DTYPE_BF16)
    return fail(FA_E_UNSUPPORTED, "fa_bwd: dtype %d not supported", a->dtype);
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(FA_E_UNSUPPORTED, "fa_bwd: head_dim %d not in {64,128,256}", a->head_dim);
  if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_k < 0)
    return fail(FA_E_INVALID, "fa_bwd: negative size");
  if (a->num_heads <= 0 || a->num_heads_k <= 0 || a->num_heads % a->num_heads_k != 0)
    return fail(FA_E_INVALID, "fa_bwd: num_heads %d not a multiple of num_heads_k %d",
                a->num_heads, a->num_heads_k);
  const void* ptrs[] = {a->q, a->k, a->v, a->out, a->dout, a->dq, a->dk, a->dv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(FA_E_UNSUPPORTED, "fa_bwd: tensors must be 16-byte aligned");
  const int64_t* strides[] = {a->q_stride,  a->k_stride,  a->v_stride,  a->o_stride,
                              a->do_stride, a->dq_stride, a->dk_stride, a->dv_stride};
  for (const int64_t* s : strides) {
    if (!strides_ok(s, 3))
      return fail(FA_E_UNSUPPORTED, "fa_bwd: strides must be non-negative multiples of 8");
    if (s[1] >= kMaxRowStride)
      return fail(FA_E_UNSUPPORTED, "fa_bwd: sequence strides must be below 2^26 elements");
  }
  if (a->has_window && (a->window_left < -1 || a->window_right < -1))
    return fail(FA_E_INVALID, "fa_bwd: window sizes must be >= -1");
  // Every grid is one-dimensional: at most one workgroup per 32 rows or keys
  // of each (batch, head), and the kernels index (batch, head, 32-row block)
  // with 32-bit integers (the row statistics' waves round that count up to a
  // multiple of 16: the margin keeps those indices in range).
  const int64_t bh = (int64_t)a->batch * a->num_heads;
  const int64_t blocks32 = ((int64_t)std::max(a->seqlen_q, a->seqlen_k) + 31) / 32;
  const int64_t rows = bh * a->seqlen_q;
  if (bh * std::max<int64_t>(blocks32, 1) > kIntMax - 64 || rows / 16 > kIntMax)
    return fail(FA_E_UNSUPPORTED, "fa_bwd: problem too large");
  return ok();
}

size_t fa_bwd_workspace_bytes(const fa_bwd_args* a) {
  if (check_bwd(a) != FA_OK) return 0;
  return fa::bwd_workspace_bytes(*a);
}

size_t fa_bwd_min_workspace_bytes(const fa_bwd_args* a) {
  if (check_bwd(a) != FA_OK) return 0;
  return fa::bwd_min_workspace_bytes(*a);
}

int fa_bwd(const fa_bwd_args* a, void* ws, size_t ws_bytes, void* stream) {
  const int st = check_bwd(a);
  if (st != FA_OK) return st;
  // seqlen_k == 0 with queries present still runs: dq is written as zero.
  if (a->batch == 0 || a->seqlen_q == 0) return ok();
  const size_t need = fa::bwd_min_workspace_bytes(*a);
  if (!ws || ws_bytes < need || !aligned16(ws))
    return fail(FA_E_WORKSPACE, "fa_bwd: workspace needs %zu bytes (16-byte aligned), got %zu",
                need, ws ? ws_bytes : (size_t)0);
  return hip_status(fa::launch_bwd(*a, ws, ws_bytes, static_cast<hipStream_t>(stream)),
                    "fa_bwd launch");
}

// ------------------------------------------------------------------ paged

static int check_paged(const fa_paged_args* a) {
  if (!a) return fail(FA_E_INVALID, "fa_paged_prefill: null args");
  if (!a->q || !a->k_cache || !a->v_cache || !a->out || !a->block_table || !a->seq_lens ||
      !a->query_start_loc || !a->prefix_kv_lens)
    return fail(FA_E_INVALID, "fa_paged_prefill: null pointer");
  if (a->dtype != FA_DTYPE_F16 && a->dtype != FA_DTYPE_BF16)
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill: dtype %d not supported", a->dtype);
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256 && a->head_dim != 512)
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill: head_dim %d not in {64,128,256,512}",
                a->head_dim);
  if (a->batch < 0 || a->num_tokens < 0 || a->max_blocks < 0 || a->num_pages < 0)
    return fail(FA_E_INVALID, "fa_paged_prefill: negative size");
  if (a->num_heads <= 0 || a->num_kv_heads <= 0 || a->num_heads % a->num_kv_heads != 0)
    return fail(FA_E_INVALID, "fa_paged_prefill: num_heads %d not a multiple of num_kv_heads %d",
                a->num_heads, a->num_kv_heads);
  if (!pow2(a->page_size))
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill: page_size %d is not a power of two",
                a->page_size);
  if (a->block_table_stride < a->max_blocks)
    return fail(FA_E_INVALID, "fa_paged_prefill: block_table_stride < max_blocks");
  if (!aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache) ||
      !aligned16(a->out))
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill: tensors must be 16-byte aligned");
  if (!strides_ok(a->q_stride, 2) || !strides_ok(a->o_stride, 2) ||
      !strides_ok(a->k_stride, 3) || !strides_ok(a->v_stride, 3))
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill: strides must be non-negative multiples of 8");
  const int64_t rows = (int64_t)a->num_tokens * (a->num_heads / a->num_kv_heads);
  if ((rows + 127) / 128 + a->batch > kIntMax / a->num_kv_heads ||
      (int64_t)a->max_blocks * a->page_size > kIntMax)
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill: problem too large");
  return ok();
}

int fa_paged_prefill(const fa_paged_args* a, void* stream) {
  const int st = check_paged(a);
  if (st != FA_OK) return st;
  if (a->batch == 0 || a->num_tokens == 0) return ok();
  if (a->num_pages == 0) return fail(FA_E_INVALID, "fa_paged_prefill: empty KV cache");
  return hip_status(fa::launch_paged_prefill(*a, static_cast<hipStream_t>(stream)),
                    "fa_paged_prefill launch");
}

int fa_paged_prefill_num_splits(const fa_paged_args* a) {
  const int st = check_paged(a);
  if (st != FA_OK) return st;
  if (a->batch == 0 || a->num_tokens == 0) return 1;
  return fa::paged_num_splits(*a);
}

static int check_splits(const fa_paged_args* a, int num_splits) {
  if (num_splits < 1 || num_splits > fa::kMaxPagedSplits)
    return fail(FA_E_INVALID, "fa_paged_prefill_splitkv: num_splits %d not in [1, %d]",
                num_splits, fa::kMaxPagedSplits);
  const int64_t grid = (int64_t)fa::paged_grid_slots(*a) * a->num_kv_heads * num_splits;
  if (grid > kIntMax)
    return fail(FA_E_UNSUPPORTED, "fa_paged_prefill_splitkv: problem too large");
  return ok();
}

size_t fa_paged_prefill_splitkv_workspace_bytes(const fa_paged_args* a, int num_splits) {
  if (check_paged(a) != FA_OK || check_splits(a, num_splits) != FA_OK) return 0;
  return fa::paged_split_workspace_bytes(*a, num_splits);
}

int fa_paged_prefill_splitkv(const fa_paged_args* a, int num_splits, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int st = check_paged(a);
  if (st != FA_OK) return st;
  st = check_splits(a, num_splits);
  if (st != FA_OK) return st;
  if (a->batch == 0 || a->num_tokens == 0) return ok();
  if (a->num_pages == 0) return fail(FA_E_INVALID, "fa_paged_prefill_splitkv: empty KV cache");
  const size_t need = fa::paged_split_workspace_bytes(*a, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(FA_E_WORKSPACE,
                "fa_paged_prefill_splitkv: workspace needs %zu bytes (16-byte aligned), got %zu",
                need, workspace ? workspace_bytes : (size_t)0);
  return hip_status(fa::launch_paged_prefill_split(*a, num_splits, workspace,
                                                   static_cast<hipStream_t>(stream)),
                    "fa_paged_prefill_splitkv launch");
}

// ------------------------------------------------------------------ decode

static int check_decode(const fa_decode_args* a) {
  if (!a) return fail(FA_E_INVALID, "fa_paged_decode: null args");
  if (!a->q || !a->k_cache || !a->v_cache || !a->out || !a->block_table || !a->seq_lens)
    return fail(FA_E_INVALID, "fa_paged_decode: null pointer");
  if (a->dtype != FA_DTYPE_F16 && a->dtype != FA_DTYPE_BF16)
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: dtype %d not supported", a->dtype);
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256 &&
      a->head_dim != 512)
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: head_dim %d not in {64,128,256,512}",
                a->head_dim);
  if (a->batch < 0 || a->max_blocks < 0 || a->max_seq_len < 0 || a->num_pages < 0)
    return fail(FA_E_INVALID, "fa_paged_decode: negative size");
  if (a->num_heads <= 0 || a->num_kv_heads <= 0 || a->num_heads % a->num_kv_heads != 0)
    return fail(FA_E_INVALID, "fa_paged_decode: num_heads %d not a multiple of num_kv_heads %d",
                a->num_heads, a->num_kv_heads);
  if (!pow2(a->page_size))
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: page_size %d is not a power of two",
                a->page_size);
  if (a->block_table_stride < a->max_blocks)
    return fail(FA_E_INVALID, "fa_paged_decode: block_table_stride < max_blocks");
  if ((int64_t)a->max_seq_len < (int64_t)a->max_blocks * a->page_size)
    return fail(FA_E_INVALID,
                "fa_paged_decode: max_seq_len %d below max_blocks * page_size", a->max_seq_len);
  if (!aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: tensors must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(a->out) & 3u) != 0 || (a->o_stride[0] & 1) ||
      (a->o_stride[1] & 1))
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: out must be 4-byte aligned");
  if (!strides_ok(a->q_stride, 2) || !strides_ok(a->k_stride, 3) || !strides_ok(a->v_stride, 3) ||
      a->o_stride[0] < 0 || a->o_stride[1] < 0)
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: unsupported strides");
  // Work items and partial rows are counted in int on the device.
  const int64_t nsplit = fa::decode_num_splits(*a);
  if (nsplit * a->num_heads * a->batch > kIntMax)
    return fail(FA_E_UNSUPPORTED, "fa_paged_decode: problem too large");
  return ok();
}

size_t fa_decode_workspace_bytes(const fa_decode_args* a) {
  if (check_decode(a) != FA_OK) return 0;
  return fa::decode_workspace_bytes(*a);
}

int fa_paged_decode(const fa_decode_args* a, void* ws, size_t ws_bytes, void* stream) {
  const int st = check_decode(a);
  if (st != FA_OK) return st;
  if (a->batch == 0) return ok();
  if (a->num_pages == 0) return fail(FA_E_INVALID, "fa_paged_decode: empty KV cache");
  const size_t need = fa::decode_workspace_bytes(*a);
  if (!ws || ws_bytes < need || !aligned16(ws))
    return fail(FA_E_WORKSPACE,
                "fa_paged_decode: workspace needs %zu bytes (16-byte aligned), got %zu", need,
                ws ? ws_bytes : (size_t)0);
  return hip_status(fa::launch_decode(*a, ws, static_cast<hipStream_t>(stream)),
                    "fa_paged_decode launch");
}

// Same validation and kernels as fa_paged_decode; the workspace is the
// device's static scratch array (no allocation, no workspace argument).
int fa_paged_decode_noalloc(const fa_decode_args* a, void* stream) {
  const int st = check_decode(a);
  if (st != FA_OK) return st;
  if (a->batch == 0) return ok();
  if (a->num_pages == 0) return fail(FA_E_INVALID, "fa_paged_decode_noalloc: empty KV cache");
  const size_t need = fa::decode_workspace_bytes(*a);
  if (need > (size_t)FA_NOALLOC_SCRATCH_BYTES)
    return fail(FA_E_WORKSPACE,
                "fa_paged_decode_noalloc: this problem needs %zu bytes of split-KV scratch, "
                "above the %zu-byte static buffer; call fa_paged_decode with a workspace",
                need, (size_t)FA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const hipError_t e = fa::noalloc_scratch(&ws);
  if (e != hipSuccess || !ws) return hip_status(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                "fa_paged_decode_noalloc scratch lookup");
  return hip_status(fa::launch_decode(*a, ws, static_cast<hipStream_t>(stream)),
                    "fa_paged_decode_noalloc launch");
}

// ------------------------------------------------------------------ cache write

static int check_cache_write(const fa_cache_write_args* a) {
  if (!a) return fail(FA_E_INVALID, "fa_reshape_and_cache: null args");
  if (!a->key || !a->value || !a->k_cache || !a->v_cache || !a->slot_mapping)
    return fail(FA_E_INVALID, "fa_reshape_and_cache: null pointer");
  if (a->dtype != FA_DTYPE_F16 && a->dtype != FA_DTYPE_BF16)
    return fail(FA_E_UNSUPPORTED, "fa_reshape_and_cache: dtype %d not supported", a->dtype);
  if (a->head_dim <= 0 || (a->head_dim & 7) != 0 || a->head_dim > 1024)
    return fail(FA_E_UNSUPPORTED, "fa_reshape_and_cache: head_dim %d not a multiple of 8 in "
                "[8, 1024]", a->head_dim);
  if (a->num_tokens < 0 || a->num_kv_heads <= 0 || a->num_pages < 0 || a->page_size <= 0)
    return fail(FA_E_INVALID, "fa_reshape_and_cache: bad size");
  if (!aligned16(a->key) || !aligned16(a->value) || !aligned16(a->k_cache) ||
      !aligned16(a->v_cache))
    return fail(FA_E_UNSUPPORTED, "fa_reshape_and_cache: tensors must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(a->slot_mapping) & 7u) != 0)
    return fail(FA_E_INVALID, "fa_reshape_and_cache: slot_mapping must be 8-byte aligned");
  if (!strides_ok(a->key_stride, 2) || !strides_ok(a->value_stride, 2) ||
      !strides_ok(a->k_stride, 3) || !strides_ok(a->v_stride, 3))
    return fail(FA_E_UNSUPPORTED,
                "fa_reshape_and_cache: strides must be non-negative multiples of 8");
  return ok();
}

int fa_reshape_and_cache(const fa_cache_write_args* a, void* stream) {
  const int st = check_cache_write(a);
  if (st != FA_OK) return st;
  if (a->num_tokens == 0 || a->num_pages == 0) return ok();
  return hip_status(fa::launch_cache_write(*a, static_cast<hipStream_t>(stream)),
                    "fa_reshape_and_cache launch");
}

}  // extern "C"
