/*
 * fa355.h — C ABI of the MI355X (gfx950) FlashAttention library `libfa355.so`.
 *
 * Every entry point takes plain device pointers, element strides and sizes.
 * The library never allocates or frees device memory and never synchronises
 * the host: the caller owns every buffer (outputs, LSE, workspaces) and passes
 * the HIP stream the work is enqueued on.  All tensors are in device memory;
 * the last (head_dim) dimension of every tensor must be contiguous.
 *
 * Return value: FA_OK (0) on success, a negative fa_status on failure.  All
 * argument checks run before any launch, so an error leaves device memory
 * untouched.  fa_strerror() gives a message for the last error on the calling
 * thread (fa_last_error_message) or a generic one for a status code.
 *
 * Reference interfaces replaced (haohervchb/Tilelang-FA-V100):
 *   fa_fwd            <- tilelang_forward_lse(...)(q, k, v) -> (out, lse)
 *                        tilelang_fa_v100/_kernels_forward.py:94-172,188-193,
 *                        called from tilelang_fa_v100/interface.py:35-36
 *   fa_bwd            <- tilelang_backward(Q, K, V, O, dO, lse, is_causal)
 *                        tilelang_fa_v100/_kernels_backward.py:200-208,
 *                        called from tilelang_fa_v100/interface.py:52
 *   fa_paged_prefill  <- get_paged_kernel(...)(q, k_cache, v_cache, block_table,
 *                        seq_lens, query_start_loc, prefix_kv_lens,
 *                        max_tokens, sm_scale)
 *                        tilelang_fa_v100/_kernels_paged.py:193-344,367-386,
 *                        called from tilelang_fa_v100/_paged_adapter.py:40-46
 *   fa_paged_decode   <- get_decode_kernel(...)(q, k_cache, v_cache,
 *                        block_table, seq_lens)
 *                        tilelang_fa_v100/_kernels_paged.py:393-516,
 *                        called from tilelang_fa_v100/_decode_adapter.py:46
 */
#ifndef FA355_H
#define FA355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 3: fa_bwd_min_workspace_bytes; fa_bwd_workspace_bytes includes the dS tiles. */
#define FA355_ABI_VERSION 3

typedef enum fa_status {
  FA_OK = 0,
  FA_E_INVALID = -1,     /* bad argument: null pointer, shape, stride, size */
  FA_E_UNSUPPORTED = -2, /* valid but not implemented: head_dim, dtype, ... */
  FA_E_HIP = -3,         /* a HIP runtime call failed (launch error)         */
  FA_E_WORKSPACE = -4    /* workspace pointer missing or too small           */
} fa_status;

typedef enum fa_dtype {
  FA_DTYPE_F16 = 0,  /* IEEE binary16 */
  FA_DTYPE_BF16 = 1  /* bfloat16      */
} fa_dtype;

/* ------------------------------------------------------------------------ */
/* Dense attention, FA2 layout q/k/v/out [batch, seqlen, heads, head_dim].   */
/* Strides are in elements: {batch, seq, head}; head_dim is contiguous;    */
/* k / v sequence strides below 2^24 elements.                             */
/* Causal masking is bottom-right aligned: key j is visible to query i iff  */
/* j <= i + seqlen_k - seqlen_q (tests/test_compare_ref.py:22 convention).  */
/* Sliding window (FlashAttention-2 window_size, off = seqlen_k - seqlen_q),*/
/* read only when has_window is non-zero (a zeroed struct has no window):   */
/* key j is visible to query i iff j >= i + off - window_left (when         */
/* window_left >= 0) and j <= i + off + window_right (when window_right     */
/* >= 0); causal implies window_right = 0.  -1 means unbounded.             */
/* A query row with no visible key gets out = 0 and lse = -inf.             */
/* ------------------------------------------------------------------------ */
typedef struct fa_fwd_args {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse; /* [batch, num_heads, seqlen_q] fp32 natural-log LSE, or NULL */
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  int32_t batch;
  int32_t seqlen_q;
  int32_t seqlen_k;
  int32_t num_heads;   /* query heads                                    */
  int32_t num_heads_k; /* key/value heads; num_heads % num_heads_k == 0 */
  int32_t head_dim;    /* 64, 128 or 256                                 */
  float softmax_scale;
  int32_t causal;
  int32_t dtype;       /* fa_dtype; q, k, v, out share it */
  int32_t has_window;   /* 0: window_left / window_right are ignored */
  int32_t window_left;  /* -1: unbounded */
  int32_t window_right; /* -1: unbounded (0 implied when causal) */
} fa_fwd_args;

/* Replaces tilelang_forward_lse (_kernels_forward.py:188-193) + the launch at
 * interface.py:35-36, without the layout copies of interface.py:19-21,38. */
int fa_fwd(const fa_fwd_args* args, void* stream);

/* Backward: LSE-recompute FlashAttention-2 gradient.  dq/dk/dv use the same
 * layout rules as q/k/v.  The workspace holds the per-row statistics (LSE and
 * dot(O, dO)) and, at head_dim 128 or 256 with causal or full attention, the 16-bit
 * dS tiles from which dq is formed (2 bytes per (query, key) pair the mask
 * lets through, up to 4 GiB); fa_bwd_workspace_bytes gives that size.  A
 * workspace of at least fa_bwd_min_workspace_bytes (the statistics only)
 * selects the path that recomputes S and dP for dq instead; both paths are
 * deterministic. */
typedef struct fa_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  const float* lse; /* [batch, num_heads, seqlen_q] as written by fa_fwd */
  void* dq;
  void* dk;
  void* dv;
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  int64_t do_stride[3];
  int64_t dq_stride[3];
  int64_t dk_stride[3];
  int64_t dv_stride[3];
  int32_t batch;
  int32_t seqlen_q;
  int32_t seqlen_k;
  int32_t num_heads;
  int32_t num_heads_k; /* num_heads % num_heads_k == 0 (GQA) */
  int32_t head_dim;    /* 64, 128 or 256 */
  float softmax_scale;
  int32_t causal;
  int32_t dtype;
  int32_t deterministic; /* accepted and ignored, as in the reference
                          * (interface.py:16-17): the backward has no atomics
                          * (each dq row is summed by one wave in a fixed
                          * order), so dq, dk and dv always repeat bit for bit,
                          * like the reference's kernels
                          * (_kernels_backward.py:10-85,88-176) */
  int32_t has_window;    /* as in fa_fwd_args */
  int32_t window_left;
  int32_t window_right;
} fa_bwd_args;

/* Replaces tilelang_backward (_kernels_backward.py:200-208). */
size_t fa_bwd_workspace_bytes(const fa_bwd_args* args);
/* No counterpart in the reference (its backward allocates its own row_dot
 * buffer, _kernels_backward.py:203): the smallest workspace fa_bwd accepts,
 * for callers that trade the dS tiles' memory for recomputing S and dP. */
size_t fa_bwd_min_workspace_bytes(const fa_bwd_args* args);
int fa_bwd(const fa_bwd_args* args, void* workspace, size_t workspace_bytes,
           void* stream);

/* ------------------------------------------------------------------------ */
/* Paged (vLLM) varlen attention.                                           */
/*   q, out      [num_tokens, num_heads, head_dim]  (strides {token, head}) */
/*   k/v_cache   [num_pages, page_size, num_kv_heads, head_dim]             */
/*               (strides {page, slot, head})                               */
/*   block_table int32 [batch, block_table_stride>=max_blocks]              */
/*   seq_lens    int32 [batch]    total KV length of each sequence          */
/*   query_start_loc int32 [batch+1]                                        */
/*   prefix_kv_lens  int32 [batch] KV tokens that precede the first query   */
/*   lse         fp32 [num_heads, num_tokens] or NULL                       */
/* Query token t (local index within its sequence) sees key n iff           */
/*   n < seq_lens[b]  and, when causal, n <= prefix_kv_lens[b] + t, and,    */
/*   when causal and a window is set, t < n + window_q (window_q > 0) and   */
/*   n < t + window_k (window_k > 0)   (_kernels_paged.py:274-308).         */
/* Only block_table entries of pages below ceil(seq_lens[b]/page_size) are  */
/* read, so padding entries may hold any value.                             */
/* ------------------------------------------------------------------------ */
typedef struct fa_paged_args {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* out;
  float* lse;
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* query_start_loc;
  const int32_t* prefix_kv_lens;
  int64_t q_stride[2];
  int64_t o_stride[2];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t block_table_stride;
  int32_t max_blocks;  /* columns of block_table that may be read */
  int32_t num_tokens;
  int32_t batch;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;    /* 64, 128, 256 or 512 */
  int32_t page_size;   /* power of two */
  int32_t num_pages;
  float softmax_scale;
  int32_t causal;
  int32_t window_q;    /* <= 0: off */
  int32_t window_k;    /* <= 0: off */
  int32_t dtype;
} fa_paged_args;

/* Replaces the paged prefill kernel (_kernels_paged.py:193-344) driven by
 * paged_forward (_paged_adapter.py:15-52).  No workspace is needed. */
int fa_paged_prefill(const fa_paged_args* args, void* stream);

/* Split-KV paged prefill.  The keys of every sequence are cut into
 * num_splits ranges (ceil(seq_len / num_splits) rounded up to 128 keys);
 * each (query tile, KV head, range) is one workgroup writing a normalised
 * fp32 partial and its LSE to the workspace, and a combine kernel merges
 * the partials into out / lse.  For batches whose query tiles alone cannot
 * fill the GPU (few new tokens against long prefixes).  Stands in for the
 * reference's split variant (_kernels_paged.py:29-191, num_splits > 1),
 * which its configs never enable (_kernels_paged.py:353-364) and which
 * walks the splits sequentially inside one block.
 *   fa_paged_prefill_num_splits: the split count paged_forward uses for
 *     these sizes and the current device's CU count (1 = no split); reads
 *     no device data.  Negative fa_status on invalid arguments.
 *   fa_paged_prefill_splitkv_workspace_bytes: bytes for num_splits
 *     (0 for num_splits == 1 or invalid arguments).
 *   fa_paged_prefill_splitkv: num_splits in [1, 64]; 1 is fa_paged_prefill
 *     (no workspace).  Same results as fa_paged_prefill within fp32
 *     rounding of the merge. */
int fa_paged_prefill_num_splits(const fa_paged_args* args);
size_t fa_paged_prefill_splitkv_workspace_bytes(const fa_paged_args* args, int num_splits);
int fa_paged_prefill_splitkv(const fa_paged_args* args, int num_splits, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Paged decode: one query token per sequence, split-KV + LSE-merge.        */
/*   q, out [batch, num_heads, head_dim] (strides {batch, head})            */
/*   caches / block_table / seq_lens as for fa_paged_args.                  */
/*   lse    fp32 [batch, num_heads] or NULL                                 */
/* max_seq_len is an upper bound of seq_lens (for example                  */
/* max_blocks * page_size); it sizes the split grid and the workspace.      */
/* ------------------------------------------------------------------------ */
typedef struct fa_decode_args {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* out;
  float* lse;
  const int32_t* block_table;
  const int32_t* seq_lens;
  int64_t q_stride[2];
  int64_t o_stride[2];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t block_table_stride;
  int32_t max_blocks;
  int32_t max_seq_len;
  int32_t batch;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;    /* 64, 128, 256 or 512 */
  int32_t page_size;
  int32_t num_pages;
  float softmax_scale;
  int32_t dtype;
} fa_decode_args;

/* Replaces the decode kernel (_kernels_paged.py:393-489) driven by
 * decode_forward (_decode_adapter.py:15-47).  The workspace size depends on
 * the sizes and on the current device's CU count (the keys per split are
 * chosen from both), so query it with the device current that the launch
 * will use. */
size_t fa_decode_workspace_bytes(const fa_decode_args* args);
int fa_paged_decode(const fa_decode_args* args, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Size of the static device scratch behind fa_paged_decode_noalloc. */
#define FA_NOALLOC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): fa_paged_decode with its split-KV workspace taken from
 * a static device array of FA_NOALLOC_SCRATCH_BYTES per GPU (held until the
 * process ends) instead of a caller buffer.  Allocates nothing.  Problems
 * whose fa_decode_workspace_bytes exceeds FA_NOALLOC_SCRATCH_BYTES are
 * rejected with FA_E_WORKSPACE.  All calls on one GPU share its array: calls
 * that overlap on that GPU (other streams, other host threads) race and
 * must be serialised by the caller; calls on one stream are ordered. */
int fa_paged_decode_noalloc(const fa_decode_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* KV-cache write (vLLM reshape_and_cache).                                 */
/*   key, value   [num_tokens, num_kv_heads, head_dim] (strides {token, head}) */
/*   k/v_cache    [num_pages, page_size, num_kv_heads, head_dim]           */
/*                (strides {page, slot, head}), the layout fa_paged_prefill */
/*                and fa_paged_decode read                                  */
/*   slot_mapping int64 [num_tokens]: token t goes to page slot_mapping[t] / */
/*                page_size, slot slot_mapping[t] % page_size; a negative   */
/*                entry (padding) or one >= num_pages * page_size is skipped */
/* Several tokens mapped to one slot leave one of them there (unspecified   */
/* which).                                                                  */
/* ------------------------------------------------------------------------ */
typedef struct fa_cache_write_args {
  const void* key;
  const void* value;
  void* k_cache;
  void* v_cache;
  const int64_t* slot_mapping;
  int64_t key_stride[2];
  int64_t value_stride[2];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t head_dim;    /* multiple of 8, at most 1024 */
  int32_t page_size;   /* > 0 */
  int32_t num_pages;
  int32_t dtype;       /* fa_dtype of key, value and both caches */
} fa_cache_write_args;

/* No counterpart in the reference, which only reads this layout
 * (_kernels_paged.py:198-199); it is the producer of the paged cache format
 * (vLLM's reshape_and_cache).  No workspace. */
int fa_reshape_and_cache(const fa_cache_write_args* args, void* stream);

/* ------------------------------------------------------------------------ */
int fa_abi_version(void);
const char* fa_strerror(int status);
/* Message of the most recent failing call on this thread ("" if none). */
const char* fa_last_error_message(void);

#ifdef __cplusplus
}
#endif
#endif /* FA355_H */
