// Dense and paged (vLLM) attention forward kernels for gfx950.
//
// Dense:  replaces _forward_lse_kernel_func (tilelang_fa_v100/
//         _kernels_forward.py:94-172).  q/k/v/out are read and written in the
//         caller's [B, S, H, D] layout through strides, so the four layout
//         copies of interface.py:19-21,38 disappear.
// Paged:  replaces _paged_kernel_func (_kernels_paged.py:193-344).  The
//         grid is sized by total query rows, not rows x batch
//         (_paged_adapter.py:44), and each workgroup finds its sequence with a
//         scan over query_start_loc.  The Hq/Hkv query heads that share a KV
//         head are packed into one row space (row = token * G + g), so every
//         K/V tile fetched from the cache serves the whole GQA group.
#include <algorithm>

#include "fa_fwd_core.h"
#include "fa_fwd_d128.h"
#include "fa_fwd_1w.h"
#include "fa_fwd_split.h"
#include "fa_internal.h"

namespace fa {

struct DenseRows {
  const uint16_t* q;
  uint16_t* o;
  float* lse;
  const uint16_t* k;
  const uint16_t* v;
  int64_t qs, os, ks, vs;  // per-row (sequence) strides, elements
  int nrows, sk, off;      // off = seqlen_k - seqlen_q
  int wl, wr;              // window bounds (-1: unbounded); causal is wr = 0
  bool has_lse;
  // K / V rows are a base plus a row stride (below 2^24 elements, checked
  // by the launcher), so whole tiles can be DMA'd through buffer resources.
  static constexpr bool kF32Out = false;
  static constexpr bool kRowStrided = true;  // k_ptr(n + m) = k_ptr(n) + m * ks

  // Row r sees keys [r + off - wl, r + off + wr] within [0, sk).
  __device__ int kv_lo(int r) const { return wl >= 0 ? min(max(r + off - wl, 0), sk) : 0; }
  __device__ int kv_hi(int r) const {
    return wr >= 0 ? min(max(r + off + wr + 1, 0), sk) : sk;
  }
  __device__ const uint16_t* q_ptr(int r) const { return q + r * qs; }
  __device__ uint16_t* o_ptr(int r) const { return o + r * os; }
  __device__ float* lse_ptr(int r) const { return lse + r; }
  __device__ const uint16_t* k_ptr(int n) const { return k + n * ks; }
  __device__ const uint16_t* v_ptr(int n) const { return v + n * vs; }
  __device__ int64_t k_row_stride() const { return ks; }
  __device__ int64_t v_row_stride() const { return vs; }
};

// Tile geometry per head_dim and core: D = 128 (both schedules) uses the
// direct-to-LDS 8-wave cores, D = 256 with PP the direct-to-LDS one-pass
// 4-wave core, the rest the register-staged 4-wave core.
template <int D, bool PP>
struct FwdKernelCfg {
  static constexpr int BM = FwdShape<D>::BM;
  static constexpr int THREADS = 256;
  static constexpr int WAVES_PER_EU = FwdShape<D>::kWavesPerEU;
  static constexpr int WG_PER_CU = WAVES_PER_EU;  // 4 waves: one per SIMD each
  static constexpr int LDS_BYTES = FwdShape<D>::LDS_ELEMS * 2;
};
// One-wave-per-SIMD cores (fa_fwd_1w.h).
template <int D, int RB>
struct FwdKernelCfg1W {
  using S = FwdShape1W<D, RB>;
  static constexpr int BM = S::BM;
  static constexpr int THREADS = 64 * S::NW;
  static constexpr int WAVES_PER_EU = 1;
  static constexpr int WG_PER_CU = 1;
  static constexpr int LDS_BYTES = 5 * S::TILEB;
};
template <>
struct FwdKernelCfg<256, true> : FwdKernelCfg1W<256, 1> {};
template <bool PP>
struct FwdKernelCfg<128, PP> {
  static constexpr int BM = FwdShapeD128::BM;
  static constexpr int THREADS = 512;
  static constexpr int WAVES_PER_EU = 2;
  static constexpr int WG_PER_CU = 1;
  static constexpr int LDS_BYTES = FwdShapeD128::LDS_BYTES;
};

// LDS: one array for the 4-wave core; four distinct arrays for the D = 128
// cores (see attn_fwd_tile_d128).  PP: the ping-pong D = 128 core, which
// needs 16 consecutive keys at a fixed row stride (dense rows, or pages of
// at least 16 keys) with row strides below 2^24 elements; otherwise the
// one-phase core.
template <class T, int D, bool PP, class Prob>
__device__ __forceinline__ void run_fwd_tile(const Prob& P, int row0, float scale) {
  if constexpr (D == 128) {
    constexpr int B = FwdShapeD128::LDS_ARRAY_BYTES;
    __shared__ __attribute__((aligned(16))) char k0[B], v0[B], k1[B], v1[B];
    if constexpr (PP)
      attn_fwd_tile_d128<T>(P, row0, scale, k0, v0, k1, v1);
    else
      attn_fwd_tile_d128_plain<T>(P, row0, scale, k0, v0, k1, v1);
  } else if constexpr (D == 256 && PP) {
    __shared__ __attribute__((aligned(16))) char smem[FwdKernelCfg1W<256, 1>::LDS_BYTES];
    attn_fwd_tile_1w<T, 256, 1>(P, row0, scale, smem);
  } else {
    __shared__ __attribute__((aligned(16))) uint16_t smem[FwdShape<D>::LDS_ELEMS];
    attn_fwd_tile<T, D>(P, row0, scale, smem);
  }
}

// A sequence of row tiles on one workgroup: next(P, row0) rewrites the
// problem and first row for the next tile, false after the last one.  The
// D = 128 ping-pong core overlaps each tile's output stores with the next
// tile's first loads; the other cores run the tiles one after the other,
// with a barrier between them (their last LDS reads are not followed by a
// barrier of their own).
template <class T, int D, bool PP, class Prob, class Next>
__device__ __forceinline__ void run_fwd_tiles(Prob P, int row0, float scale, Next next) {
  if constexpr (D == 128 && PP) {
    constexpr int B = FwdShapeD128::LDS_ARRAY_BYTES;
    __shared__ __attribute__((aligned(16))) char k0[B], v0[B], k1[B], v1[B];
    attn_fwd_tiles_d128<T>(P, row0, scale, k0, v0, k1, v1, next);
  } else {
    for (;;) {
      run_fwd_tile<T, D, PP>(P, row0, scale);
      if (!next(P, row0)) break;
      __syncthreads();
    }
  }
}

// MODE (MaskMode): full attention, causal, or a window band from the
// arguments.  The causal and full bands are compile-time constants.
template <class T, int D, int MODE>
__global__ __launch_bounds__((FwdKernelCfg<D, true>::THREADS),
                             (FwdKernelCfg<D, true>::WAVES_PER_EU))
void fwd_dense_kernel(fa_fwd_args a) {
  using C = FwdKernelCfg<D, true>;
  const int qtiles = (a.seqlen_q + C::BM - 1) / C::BM;
  const int nbh = a.batch * a.num_heads;
  // Persistent: this workgroup's tiles are rounds 0, 1, ... of
  // persistent_tile (one workgroup per tile when the grid covers them all).
  // Each tile's problem is set up from the arguments in the kernarg segment.
  auto setup = [qtiles, nbh](int vid, DenseRows& P, int& row0) {
    const auto* ap = kernel_args<fa_fwd_args>();
    const TileHead th = xcd_tile_order(vid, qtiles, nbh);
    const int bh = th.bh;
    const int H = ap->num_heads;
    const int h = bh % H;
    const int b = bh / H;
    // Heaviest causal tiles (largest query index) first.
    const int qt = MODE != kMaskNone ? qtiles - 1 - th.rank : th.rank;
    const int hk = h / (H / ap->num_heads_k);
    P.q = static_cast<const uint16_t*>(ap->q) + b * ap->q_stride[0] + h * ap->q_stride[2];
    P.o = static_cast<uint16_t*>(ap->out) + b * ap->o_stride[0] + h * ap->o_stride[2];
    P.lse = ap->lse ? ap->lse + ((int64_t)b * H + h) * ap->seqlen_q : nullptr;
    P.k = static_cast<const uint16_t*>(ap->k) + b * ap->k_stride[0] + hk * ap->k_stride[2];
    P.v = static_cast<const uint16_t*>(ap->v) + b * ap->v_stride[0] + hk * ap->v_stride[2];
    P.qs = ap->q_stride[1];
    P.os = ap->o_stride[1];
    P.ks = ap->k_stride[1];
    P.vs = ap->v_stride[1];
    P.nrows = ap->seqlen_q;
    P.sk = ap->seqlen_k;
    P.off = ap->seqlen_k - ap->seqlen_q;
    const Band band = mode_band<MODE>(*ap);
    P.wl = band.wl;
    P.wr = band.wr;
    P.has_lse = ap->lse != nullptr;
    row0 = qt * C::BM;
  };
  DenseRows P;
  int row0 = 0;
  if constexpr (MODE == kMaskBand) {
    // A band from the arguments costs the core registers (the tile loop
    // around it spilled inside the key loop): one workgroup per tile.
    if (blockIdx.x >= (unsigned)(qtiles * nbh)) return;
    setup(blockIdx.x, P, row0);
    run_fwd_tile<T, D, true>(P, row0, a.softmax_scale);
    return;
  }
  int r = 0;
  const int vid = persistent_tile(blockIdx.x, gridDim.x, r, qtiles * nbh, nbh);
  if (vid < 0) return;
  setup(vid, P, row0);
  run_fwd_tiles<T, D, true>(P, row0, a.softmax_scale, [&](DenseRows& Pn, int& rn) {
    const int v = persistent_tile(blockIdx.x, gridDim.x, ++r, qtiles * nbh, nbh);
    if (v < 0) return false;
    setup(v, Pn, rn);
    return true;
  });
}

struct PagedRows {
  const uint16_t* q;  // token 0 of the sequence, head hk*G
  uint16_t* o;
  float* lse;         // [Hq, num_tokens] at head hk*G, token 0 of the sequence
  int64_t q_tok, q_head, o_tok, o_head, lse_head;
  const uint16_t* kc;  // head hk
  const uint16_t* vc;
  int64_t k_page, k_slot, v_page, v_slot;
  const int32_t* bt;   // block_table row of the sequence
  int ps_log2, ps_mask, last_page;
  int G, nrows, seq_len, prefix, wq, wk;
  bool causal, has_lse;
  static constexpr bool kF32Out = false;
  static constexpr bool kRowStrided = false;

  __device__ int kv_lo(int r) const {
    if (!causal || wq <= 0) return 0;
    return max(0, r / G - wq + 1);
  }
  __device__ int kv_hi(int r) const {
    const int t = r / G;
    int hi = seq_len;
    if (causal) hi = min(hi, prefix + t + 1);
    if (causal && wk > 0) hi = min(hi, t + wk);
    return hi;
  }
  __device__ const uint16_t* q_ptr(int r) const {
    const int t = r / G;
    return q + t * q_tok + (r - t * G) * q_head;
  }
  __device__ uint16_t* o_ptr(int r) const {
    const int t = r / G;
    return o + t * o_tok + (r - t * G) * o_head;
  }
  __device__ float* lse_ptr(int r) const {
    const int t = r / G;
    return lse + (r - t * G) * lse_head + t;
  }
  __device__ int64_t page_of(int n) const {
    // The block table is read-only for the kernel's lifetime: through a
    // constant-address-space pointer a wave-uniform n reads it with a scalar
    // load (waited for on lgkmcnt).  A plain load compiled to a vector load
    // followed by vmcnt(0), which also waited for every K / V tile DMA in
    // flight, twice per tile.  The clamp guards against a corrupt table;
    // valid tables are unaffected.
    const auto* btc = (const __attribute__((address_space(4))) int32_t*)bt;
    return (int64_t)min((unsigned)btc[n >> ps_log2], (unsigned)last_page);
  }
  __device__ const uint16_t* k_ptr(int n) const {
    return kc + page_of(n) * k_page + (n & ps_mask) * k_slot;
  }
  __device__ const uint16_t* v_ptr(int n) const {
    return vc + page_of(n) * v_page + (n & ps_mask) * v_slot;
  }
  // Stride between consecutive keys of one page.
  __device__ int64_t k_row_stride() const { return k_slot; }
  __device__ int64_t v_row_stride() const { return v_slot; }
};

// One split of a split-KV paged prefill: the keys of the sequence are cut
// into nsplit ranges of a multiple of 128 keys; this problem sees only keys
// in [split_lo, split_hi) and writes its normalised partial O (fp32) and
// base-2 LSE into the workspace at [split][head][token].
struct PagedSplitRows : PagedRows {
  static constexpr bool kF32Out = true;
  int split_lo, split_hi;
  float* po;     // [nsplit][Hq][num_tokens][D] at (split, head hk*G, token 0 of the sequence)
  float* plse;   // [nsplit][Hq][num_tokens]    at the same origin
  int64_t p_head;  // num_tokens
  int D;

  __device__ int kv_lo(int r) const { return max(PagedRows::kv_lo(r), split_lo); }
  __device__ int kv_hi(int r) const { return min(PagedRows::kv_hi(r), split_hi); }
  __device__ float* o32_ptr(int r) const {
    const int t = r / G;
    return po + ((r - t * G) * p_head + t) * D;
  }
  __device__ float* lse2_ptr(int r) const {
    const int t = r / G;
    return plse + (r - t * G) * p_head + t;
  }
};

// Finds the sequence owning `tile` in the varlen tile space where sequence b
// has ceil(qlen_b * G / BM) tiles.  Returns b (or -1) and the tile index
// within the sequence.  Wave 0 scans the sequences 64 at a time with a
// shuffle prefix sum and finds the owner with a ballot; one barrier hands
// the result to the other waves (a block-wide scan in LDS took 16
// barriers).  Up to 64 sequences are taken in order of decreasing history
// (prefix_kv_lens; equal histories keep their order): a sequence's tiles all
// see about its history plus its own length in keys, so with the
// heaviest-first order inside each sequence the tiles go out roughly
// longest first, and the last workgroups on each CU are short (C5, chunked
// prefill with histories of 0-8k keys: 2% faster; 5% less idle time in a
// dispatch simulation, part of it spent on the sort).  When all histories
// are equal the order is the sequences' own.
__device__ int find_sequence(const int32_t* qsl, const int32_t* prefix, int batch, int G,
                             int BM, int tile, int* local) {
  __shared__ int found_b, found_local;
  if (wave_id() == 0) {
    const int lane = threadIdx.x & 63;
    int base = 0, fb = -1, fl = 0;
    // The sort costs wave 0 about a microsecond of dependent shuffles; it is
    // skipped when the histories are all equal (the order would not change).
    const bool sort = batch <= 64 &&
                      __ballot(lane < batch && prefix[lane] != prefix[0]) != 0;
    if (sort) {
      // Bitonic sort of (history descending, index ascending) across lanes;
      // lanes past the batch sort last.
      const uint32_t hist = lane < batch ? (uint32_t)max(prefix[lane], 0) : 0u;
      uint64_t key = lane < batch ? ((uint64_t)(0x7fffffffu - hist) << 32) | (uint32_t)lane
                                  : ~0ull;
#pragma unroll
      for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
          const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(key >> 32), j) << 32) |
                                 (uint32_t)__shfl_xor((int)(uint32_t)key, j);
          const bool up = (lane & k) == 0, lower = (lane & j) == 0;
          const uint64_t lo = key < other ? key : other, hi = key < other ? other : key;
          key = (up == lower) ? lo : hi;
        }
      const int sb = key == ~0ull ? batch : (int)(uint32_t)key;  // sequence at this lane
      int n = 0;
      if (sb < batch) {
        const int ql = qsl[sb + 1] - qsl[sb];
        n = ql > 0 ? (int)(((int64_t)ql * G + BM - 1) / BM) : 0;
      }
      int incl = n;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
      }
      const int excl = incl - n;
      const bool hit = sb < batch && n > 0 && tile >= excl && tile < incl;
      const uint64_t m = __ballot(hit);
      if (m) {
        const int src = __ffsll((unsigned long long)m) - 1;
        fb = __shfl(sb, src);
        fl = tile - __shfl(excl, src);
      }
    } else {
      for (int c0 = 0; c0 < batch; c0 += 64) {
        const int b = c0 + lane;
        int n = 0;
        if (b < batch) {
          const int ql = qsl[b + 1] - qsl[b];
          n = ql > 0 ? (int)(((int64_t)ql * G + BM - 1) / BM) : 0;
        }
        int incl = n;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int v = __shfl_up(incl, off);
          if (lane >= off) incl += v;
        }
        const int excl = incl - n;
        const bool hit = b < batch && n > 0 && tile >= base + excl && tile < base + incl;
        const uint64_t m = __ballot(hit);
        if (m) {
          const int src = __ffsll((unsigned long long)m) - 1;
          fb = c0 + src;
          fl = tile - base - __shfl(excl, src);
          break;
        }
        base += __shfl(incl, 63);
      }
    }
    if (lane == 0) {
      found_b = fb;
      found_local = fl;
    }
  }
  __syncthreads();
  *local = found_local;
  return found_b;
}

// Row problem of KV head hk of sequence b (query tokens qs .. qs+qlen-1).
__device__ __forceinline__ void paged_rows(const fa_paged_args& a, int hk, int b, int qs,
                                           int qlen, PagedRows& P) {
  const int G = a.num_heads / a.num_kv_heads;
  P.G = G;
  P.nrows = qlen * G;
  P.q = static_cast<const uint16_t*>(a.q) + (int64_t)qs * a.q_stride[0] +
        (int64_t)hk * G * a.q_stride[1];
  P.o = static_cast<uint16_t*>(a.out) + (int64_t)qs * a.o_stride[0] +
        (int64_t)hk * G * a.o_stride[1];
  P.q_tok = a.q_stride[0];
  P.q_head = a.q_stride[1];
  P.o_tok = a.o_stride[0];
  P.o_head = a.o_stride[1];
  P.has_lse = a.lse != nullptr;
  P.lse = a.lse ? a.lse + (int64_t)hk * G * a.num_tokens + qs : nullptr;
  P.lse_head = a.num_tokens;
  P.kc = static_cast<const uint16_t*>(a.k_cache) + (int64_t)hk * a.k_stride[2];
  P.vc = static_cast<const uint16_t*>(a.v_cache) + (int64_t)hk * a.v_stride[2];
  P.k_page = a.k_stride[0];
  P.k_slot = a.k_stride[1];
  P.v_page = a.v_stride[0];
  P.v_slot = a.v_stride[1];
  P.bt = a.block_table + (int64_t)b * a.block_table_stride;
  P.ps_log2 = __builtin_ctz(a.page_size);
  P.ps_mask = a.page_size - 1;
  P.last_page = a.num_pages - 1;
  // Keys beyond the block table's reach cannot be resolved; they are treated
  // as absent.
  P.seq_len = max(0, min(a.seq_lens[b], a.max_blocks * a.page_size));
  P.prefix = a.prefix_kv_lens[b];
  P.causal = a.causal != 0;
  P.wq = a.window_q;
  P.wk = a.window_k;
}

template <class T, int D, bool PP>
__global__ __launch_bounds__((FwdKernelCfg<D, PP>::THREADS), (FwdKernelCfg<D, PP>::WAVES_PER_EU))
void fwd_paged_kernel(fa_paged_args a) {
  using S = FwdKernelCfg<D, PP>;
  const int G = a.num_heads / a.num_kv_heads;
  const int slots = gridDim.x / a.num_kv_heads;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int hk = id / slots;
  const int slot = id % slots;

  int local = 0;
  const int b = find_sequence(a.query_start_loc, a.prefix_kv_lens, a.batch, G, S::BM, slot, &local);
  if (b < 0) return;
  const int qs = a.query_start_loc[b];
  const int qlen = a.query_start_loc[b + 1] - qs;
  const int ntiles = (int)(((int64_t)qlen * G + S::BM - 1) / S::BM);
  // Later tiles of a causal sequence see more keys: run them first.
  const int tile = ntiles - 1 - local;
  PagedRows P;
  paged_rows(a, hk, b, qs, qlen, P);
  run_fwd_tile<T, D, PP>(P, tile * S::BM, a.softmax_scale);
}

// Split-KV variant: workgroup (split, KV head, tile slot); the splits of a
// sequence cover its keys in ranges of ceil(seq_len / nsplit) rounded up to
// 128.  Consecutive workgroup ids share the split and KV head (the same
// K / V pages).
template <class T, int D, bool PP>
__global__ __launch_bounds__((FwdKernelCfg<D, PP>::THREADS), (FwdKernelCfg<D, PP>::WAVES_PER_EU))
void fwd_paged_split_kernel(fa_paged_args a, int nsplit, float* po, float* plse) {
  using S = FwdKernelCfg<D, PP>;
  const int G = a.num_heads / a.num_kv_heads;
  const int per_split = gridDim.x / nsplit;
  const int slots = per_split / a.num_kv_heads;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int split = id / per_split;
  const int hk = (id % per_split) / slots;
  const int slot = id % slots;

  int local = 0;
  const int b = find_sequence(a.query_start_loc, a.prefix_kv_lens, a.batch, G, S::BM, slot, &local);
  if (b < 0) return;
  const int qs = a.query_start_loc[b];
  const int qlen = a.query_start_loc[b + 1] - qs;
  const int ntiles = (int)(((int64_t)qlen * G + S::BM - 1) / S::BM);
  const int tile = ntiles - 1 - local;
  PagedSplitRows P;
  paged_rows(a, hk, b, qs, qlen, P);
  const int chunk = ((P.seq_len + nsplit - 1) / nsplit + 127) / 128 * 128;
  P.split_lo = split * chunk;
  P.split_hi = P.split_lo + chunk;
  const int64_t origin = ((int64_t)split * a.num_heads + (int64_t)hk * G) * a.num_tokens + qs;
  P.po = po + origin * D;
  P.plse = plse + origin;
  P.p_head = a.num_tokens;
  P.D = D;
  run_fwd_tile<T, D, PP>(P, tile * S::BM, a.softmax_scale);
}

// Merges the nsplit partials of each (query head, token): O = sum_s w_s O_s /
// sum_s w_s with w_s = 2^(lse_s - max); LSE = ln 2 (max + log2 sum_s w_s).
// One wave per (head, token); tokens outside query_start_loc[0] ..
// query_start_loc[batch] belong to no sequence and are left untouched, as
// the unsplit kernel leaves them.
template <class T, int D>
__global__ __launch_bounds__(256) void paged_combine_kernel(fa_paged_args a, int nsplit,
                                                            const float* po,
                                                            const float* plse) {
  constexpr int NP = (D + 127) / 128;  // d pairs per lane: 2 lane + 128 k
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  const int64_t NT = a.num_tokens;
  if (item >= (int64_t)a.num_heads * NT) return;
  const int h = (int)(item / NT);
  const int t = (int)(item % NT);
  if (t < a.query_start_loc[0] || t >= a.query_start_loc[a.batch]) return;
  const int64_t stride_s = (int64_t)a.num_heads * NT;  // rows per split
  const int64_t row = (int64_t)h * NT + t;
  float m = neg_inf();
  for (int s = lane; s < nsplit; s += 64) m = fmaxf(m, plse[s * stride_s + row]);
  m = wave_max(m);
  const float m_use = m == neg_inf() ? 0.f : m;
  float acc[NP][2];
#pragma unroll
  for (int k = 0; k < NP; ++k) acc[k][0] = acc[k][1] = 0.f;
  float wsum = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float ls = plse[s * stride_s + row];
    const float w = ls == neg_inf() ? 0.f : fast_exp2(ls - m_use);
    wsum += w;
    const float* src = po + (s * stride_s + row) * D;
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int d = 2 * lane + 128 * k;
      if (d < D) {
        const float2 pv = *reinterpret_cast<const float2*>(src + d);
        acc[k][0] = fmaf(w, pv.x, acc[k][0]);
        acc[k][1] = fmaf(w, pv.y, acc[k][1]);
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  uint16_t* op = static_cast<uint16_t*>(a.out) + (int64_t)t * a.o_stride[0] +
                 (int64_t)h * a.o_stride[1];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int d = 2 * lane + 128 * k;
    if (d < D)
      *reinterpret_cast<uint32_t*>(op + d) = T::pack(acc[k][0] * inv, acc[k][1] * inv);
  }
  if (a.lse && lane == 0) a.lse[row] = wsum > 0.f ? (m_use + log2f(wsum)) * kLn2 : neg_inf();
}

// ----------------------------------------------------------------- launchers

// Keys split across the waves of a workgroup (fa_fwd_split.h): one
// workgroup per 32 query rows of a head.
template <class T, int D>
static hipError_t launch_dense_split(const fa_fwd_args& a, int mode, hipStream_t st) {
  using S = FwdSplitShape<D>;
  const dim3 grid((unsigned)((a.seqlen_q + 31) / 32) * a.num_heads * a.batch),
      block(64 * S::NW);
  if (mode == kMaskCausal)
    hipLaunchKernelGGL((fwd_split_kernel<T, D, kMaskCausal>), grid, block, 0, st, a);
  else if (mode == kMaskBand)
    hipLaunchKernelGGL((fwd_split_kernel<T, D, kMaskBand>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((fwd_split_kernel<T, D, kMaskNone>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <class T, int D>
static hipError_t launch_dense(const fa_fwd_args& a, hipStream_t st) {
  using C = FwdKernelCfg<D, true>;
  const int qtiles = (a.seqlen_q + C::BM - 1) / C::BM;
  const int mode = mask_mode(a);
  if constexpr (D == 64 || D == 128) {
    // Too few query tiles to give most CUs a workgroup: split the keys.
    const int64_t wgs = (int64_t)qtiles * a.num_heads * a.batch;
    if (wgs * tiles::kFwdSplitMaxFillDen < (int64_t)device_cu_count() * tiles::kFwdSplitMaxFillNum)
      return launch_dense_split<T, D>(a, mode, st);
  }
  // Band instances run one workgroup per tile (fwd_dense_kernel).
  const bool band = mode == kMaskBand;
  const dim3 grid((unsigned)(band ? qtiles * a.num_heads * a.batch
                                  : persistent_grid(qtiles, a.num_heads * a.batch,
                                                    C::WG_PER_CU)));
  if (mode == kMaskCausal)
    hipLaunchKernelGGL((fwd_dense_kernel<T, D, kMaskCausal>), grid, dim3(C::THREADS), 0, st, a);
  else if (band)
    hipLaunchKernelGGL((fwd_dense_kernel<T, D, kMaskBand>), grid, dim3(C::THREADS), 0, st, a);
  else
    hipLaunchKernelGGL((fwd_dense_kernel<T, D, kMaskNone>), grid, dim3(C::THREADS), 0, st, a);
  return hipGetLastError();
}

template <class T>
static hipError_t dispatch_dense_d(const fa_fwd_args& a, hipStream_t st) {
  switch (a.head_dim) {
    case 64: return launch_dense<T, 64>(a, st);
    case 128: return launch_dense<T, 128>(a, st);
    case 256: return launch_dense<T, 256>(a, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fwd(const fa_fwd_args& a, hipStream_t st) {
  return a.dtype == FA_DTYPE_BF16 ? dispatch_dense_d<BFloat16>(a, st)
                                  : dispatch_dense_d<Half>(a, st);
}

// The D = 128 ping-pong core and the D = 256 core take K / V in runs of 16
// (D = 128) or 8 (D = 256) keys at a fixed row stride: pages of at least 16
// keys, token strides below 2^24 elements.
static bool paged_pingpong(const fa_paged_args& a) {
  const int64_t lim = int64_t(1) << 24;
  return (a.head_dim == 128 || a.head_dim == 256) && a.page_size >= 16 &&
         a.k_stride[1] < lim && a.v_stride[1] < lim;
}

int paged_block_rows(const fa_paged_args& a) {
  const bool pp = paged_pingpong(a);
  switch (a.head_dim) {
    case 64: return FwdKernelCfg<64, false>::BM;
    case 128: return FwdKernelCfg<128, false>::BM;
    case 256: return pp ? FwdKernelCfg<256, true>::BM : FwdKernelCfg<256, false>::BM;
    default: return FwdKernelCfg<512, false>::BM;
  }
}

int paged_grid_slots(const fa_paged_args& a) {
  const int G = a.num_heads / a.num_kv_heads;
  const int64_t rows = (int64_t)a.num_tokens * G;
  const int bm = paged_block_rows(a);
  // sum_b ceil(rows_b / BM) <= ceil(rows / BM) + batch
  return (int)((rows + bm - 1) / bm + a.batch);
}

template <class T, int D, bool PP>
static hipError_t launch_paged_pp(const fa_paged_args& a, int nsplit, void* ws,
                                  hipStream_t st) {
  const unsigned slots = (unsigned)paged_grid_slots(a) * a.num_kv_heads;
  if (nsplit <= 1) {
    hipLaunchKernelGGL((fwd_paged_kernel<T, D, PP>), dim3(slots),
                       dim3(FwdKernelCfg<D, PP>::THREADS), 0, st, a);
    return hipGetLastError();
  }
  const size_t rows = (size_t)nsplit * a.num_heads * a.num_tokens;
  float* po = static_cast<float*>(ws);
  float* plse = po + rows * D;
  hipLaunchKernelGGL((fwd_paged_split_kernel<T, D, PP>), dim3(slots * (unsigned)nsplit),
                     dim3(FwdKernelCfg<D, PP>::THREADS), 0, st, a, nsplit, po, plse);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t items = (int64_t)a.num_heads * a.num_tokens;
  hipLaunchKernelGGL((paged_combine_kernel<T, D>), dim3((unsigned)((items + 3) / 4)), dim3(256),
                     0, st, a, nsplit, po, plse);
  return hipGetLastError();
}

template <class T, int D>
static hipError_t launch_paged(const fa_paged_args& a, int nsplit, void* ws, hipStream_t st) {
  if constexpr (D == 128 || D == 256) {
    if (paged_pingpong(a)) return launch_paged_pp<T, D, true>(a, nsplit, ws, st);
  }
  return launch_paged_pp<T, D, false>(a, nsplit, ws, st);
}

template <class T>
static hipError_t dispatch_paged_d(const fa_paged_args& a, int nsplit, void* ws,
                                   hipStream_t st) {
  switch (a.head_dim) {
    case 64: return launch_paged<T, 64>(a, nsplit, ws, st);
    case 128: return launch_paged<T, 128>(a, nsplit, ws, st);
    case 256: return launch_paged<T, 256>(a, nsplit, ws, st);
    case 512: return launch_paged<T, 512>(a, nsplit, ws, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_paged_prefill(const fa_paged_args& a, hipStream_t st) {
  return launch_paged_prefill_split(a, 1, nullptr, st);
}

hipError_t launch_paged_prefill_split(const fa_paged_args& a, int nsplit, void* ws,
                                      hipStream_t st) {
  return a.dtype == FA_DTYPE_BF16 ? dispatch_paged_d<BFloat16>(a, nsplit, ws, st)
                                  : dispatch_paged_d<Half>(a, nsplit, ws, st);
}

size_t paged_split_workspace_bytes(const fa_paged_args& a, int nsplit) {
  if (nsplit <= 1) return 0;
  const size_t rows = (size_t)nsplit * a.num_heads * a.num_tokens;
  return rows * a.head_dim * sizeof(float) + rows * sizeof(float) + 256;
}

// Split count from sizes alone (no device data): split only when the query
// tiles cannot occupy the GPU (fewer workgroups than CUs) and the block
// table can hold long sequences; each split covers at least 2048 keys.
int paged_num_splits(const fa_paged_args& a) {
  const int G = a.num_heads / a.num_kv_heads;
  const int64_t tiles =
      ((int64_t)a.num_tokens * G + paged_block_rows(a) - 1) / paged_block_rows(a);
  const int64_t wgs = std::max<int64_t>(1, tiles * a.num_kv_heads);
  const int64_t kv_cap = (int64_t)a.max_blocks * a.page_size;
  const int cus = device_cu_count();
  if (wgs >= cus || kv_cap < tiles::kSplitMinKeys) return 1;
  // About one workgroup per CU, and no range longer than kSplitMaxRangeKeys
  // (a workgroup's serial length), but none shorter than kSplitMinRangeKeys
  // (each split adds a partial O per row to write and merge).
  int64_t ns = std::max<int64_t>((cus + wgs - 1) / wgs,
                                 (kv_cap + tiles::kSplitMaxRangeKeys - 1) / tiles::kSplitMaxRangeKeys);
  ns = std::min<int64_t>(ns, kv_cap / tiles::kSplitMinRangeKeys);
  return (int)std::max<int64_t>(1, std::min<int64_t>(ns, kMaxPagedSplits));
}

}  // namespace fa
