// Persistent streaming split-KV decode for head_dim 64 / 128 / 256 / 512 and
// pages of at least 16 keys, or of fewer when one DMA instruction's rows
// (1024 / 2D) still fit a page (gfx950); smaller pages take the chunked
// decode_split_kernel (fa_decode.hip).
//
// Work item = (sequence b, KV head, group of GB query heads, split c), one
// split being kSplit consecutive keys.  Items are numbered sequence-major,
// split-minor, so consecutive items continue the same key stream.  A
// workgroup holds kWavesPerWG independent waves; each wave owns a contiguous
// range of items and walks their keys in 16-key tiles:
//  * every load reads whole rows (2D bytes: D / 8 lanes per row, 1024 / 2D
//    rows per instruction) with the non-temporal hint and goes straight to
//    LDS (global_load_lds).  That pattern streams close to the HBM peak, whereas
//    64-byte pieces of 16 rows per instruction (the MFMA operand layout read
//    from global memory directly) cost about 15% of it;
//  * each wave has an LDS ring of kDepth tiles (K rows then V rows, 16-byte
//    chunks XOR-swizzled per row so the K row reads and the V transpose
//    reads avoid bank conflicts).  A tile is read into registers and its
//    slot is refilled at once, so kDepth tiles stay in flight while it is
//    computed; one fixed vmcnt wait before the operand reads replaces any
//    barrier.  Depth and waves per workgroup scale with D so that every
//    head_dim keeps about 128 KB of K / V in flight per CU;
//  * the page of a 16-key tile is wave-uniform (page size >= 16), so the
//    block table is read with scalar loads, one tile ahead of its use;
//  * S^T = K Q^T and O^T += V^T P^T both run on v_mfma_f32_16x16x32, with the
//    GB query heads as the 16 columns.  P leaves the first product in the
//    layout the second takes as its B operand (its 16 keys fill half of the
//    32-deep k dimension, the other half is zero), and V^T comes from
//    ds_read_b64_tr_b16, so the VALU only does the softmax;
//  * the running max moves only when it grows by more than 2^8 (as in the
//    prefill kernels), so O is rarely rescaled;
//  * the query rows of an item go to LDS by DMA too, issued with the item's
//    first tile when the wave's query slot is free;
//  * at the end of an item each lane writes its 32 normalised O^T values and
//    the head's base-2 LSE for the combine kernel.
// A sequence's item count is ceil(len / split) * heads / GB; the first wave
// prefix-sums these over the batch into LDS, so the grid never holds empty work.
// split (keys per item) is chosen per call by the launcher from the sizes
// (max_seq_len); the first wave doubles it when the actual lengths still give
// every wave kDecItemsPerWave items at twice the split, and workgroup 0
// records the split it used for the combine kernel.
#pragma once

#include "fa355.h"
#include "fa_common.h"

namespace fa {

template <int D_>
struct DecStream {
  static constexpr int D = D_;
  static constexpr int kSplitMax = tiles::kDecSplitKeysMax;  // keys per item, largest choice
  static constexpr int kSplitMin = tiles::kDecSplitKeysMin;  // smallest choice
  static constexpr int kTile = tiles::kDecTileKeys;        // keys per tile
  static constexpr int kMaxBatch = 1024;
  static constexpr int kMaxGroup = 8;  // query heads per item (MFMA columns used)
  static constexpr int kRowBytes = D * 2;
  static constexpr int kTileBytes = 2 * kTile * kRowBytes;  // K rows, then V rows
  static constexpr int kRowsPerDma = 1024 / kRowBytes;     // rows per DMA instruction
  static constexpr int kLanesPerRow = 64 / kRowsPerDma;    // = D / 8, the row's chunks
  static constexpr int kDmaPerTensor = kTile / kRowsPerDma;
  static constexpr int kDmaPerTile = 2 * kDmaPerTensor;
  // Tiles in flight per wave and waves per workgroup (one workgroup per CU,
  // its LDS ring is 128 KB): D = 64: 4 x 4 KB x 8 waves; 128: 2 x 8 KB x 8;
  // 256: 2 x 16 KB x 4; 512: 2 x 32 KB x 2.
  static constexpr int kDepth = D == 128 ? tiles::kDecTilesInFlight : (D == 64 ? 4 : 2);
  static constexpr int kWavesPerWG = D <= 128 ? 8 : 512 / D * 2;
  static constexpr int kWavesPerCU = kWavesPerWG;
  static constexpr int kWavesPerSimd = kWavesPerWG >= 8 ? 2 : 1;
  // Query-slot rows: GB rounded up to whole DMA instructions.
  static constexpr int kQueryRows = kMaxGroup > kRowsPerDma ? kMaxGroup : kRowsPerDma;
  static constexpr int kSwzMask = D / 8 >= 16 ? 15 : D / 8 - 1;
  static_assert(kRowsPerDma * kRowBytes == 1024 && kDmaPerTensor * kRowsPerDma == kTile, "DMA");
  static_assert(kWavesPerWG * kDepth * kTileBytes == 128 * 1024, "LDS ring");
};

struct DecodeWsS {
  float* po;    // [B, Hq, nsplit, D]
  float* plse;  // [B, Hq, nsplit]
  int* split_out;  // the split size used (written by workgroup 0)
  int nsplit;      // partials per (sequence, head) the workspace holds at `split`
  int split;       // keys per item chosen by the launcher (a multiple of kTile)
};

// Item -> (b, kv head, head group, split, key range) through the batch
// prefix sums of item counts held in LDS.
struct DecItem {
  int b, hk, hg, c, n_begin, n_end, ntiles;
};

// Read-only views in the constant address space.  The block table and the
// sequence lengths are not written while a decode kernel runs, so uniform
// reads through these views are selected as scalar loads; a vector load
// would have to wait for every K/V load issued before it.
typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
__device__ __forceinline__ const_i32_ptr as_const(const int32_t* p) {
  return (const_i32_ptr)(const __attribute__((address_space(4))) void*)(uintptr_t)p;
}

__device__ __forceinline__ DecItem dec_item(int I, const int* pfx, const_i32_ptr seq_lens, int cap,
                                            int B, int HG, int ngroups, int split) {
  const int u = I / HG, h = I - u * HG;  // unit (sequence, split), head slot
  int lo = 0, hi = B;  // largest b with pfx[b] <= u
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (pfx[mid] <= u) lo = mid; else hi = mid;
  }
  // I is wave-uniform, so every lane finds the same item: moving the fields
  // to scalar registers keeps the block-table reads on the scalar path.
  DecItem it;
  it.b = __builtin_amdgcn_readfirstlane(lo);
  const int len = max(0, min(seq_lens[it.b], cap));
  it.c = u - __builtin_amdgcn_readfirstlane(pfx[it.b]);
  it.hk = h / ngroups;
  it.hg = h % ngroups;
  it.n_begin = it.c * split;
  it.n_end = min(it.n_begin + split, len);
  it.ntiles = (it.n_end - it.n_begin + tiles::kDecTileKeys - 1) / tiles::kDecTileKeys;
  return it;
}

// 16-byte chunk c of a 256-byte row r sits at chunk position c ^ swz(r).
__device__ __forceinline__ int dec_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}

// Non-temporal 16-byte load straight to LDS (lane l writes bytes
// [16 l, 16 l + 16) after `lds`).
__device__ __forceinline__ void ld16_lds_nt(const void* g, char* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0,
                                   /*nt*/ 2);
}

// Reads one tile's operands from LDS once its loads have landed: the D / 32
// K MFMA operands and, for each of the D / 16 16-wide d blocks, the V^T
// operand (4 keys x 1 d per lane, ds_read_b64_tr_b16).  When a tile is read,
// the only vector memory operations issued after its own kDmaPerTile DMA
// instructions are the later tiles' (kDepth - 1) x kDmaPerTile, possibly a
// query-row DMA and partial-result stores; the hardware counter completes
// in order, so vmcnt((kDepth - 1) x kDmaPerTile) means the tile (and a
// query-row DMA issued before it) is resident.  The reads are opaque to the
// compiler on purpose: its tracking of LDS DMA either waits for every
// outstanding load or misses the dependence.  They are issued in groups of
// (4 K, 8 V) reads (2 and 4 at head_dim 64), each group one statement that
// ends with its own lgkmcnt(0), so no result is used before it has landed.
__device__ __forceinline__ void lds_read_k4v8(uint32_t base, const int* koff, const int* voff,
                                              u32x4* k, u32x2* v) {
  asm volatile(
      "ds_read_b128 %0, %12\n\t"
      "ds_read_b128 %1, %13\n\t"
      "ds_read_b128 %2, %14\n\t"
      "ds_read_b128 %3, %15\n\t"
      "ds_read_b64_tr_b16 %4, %16\n\t"
      "ds_read_b64_tr_b16 %5, %17\n\t"
      "ds_read_b64_tr_b16 %6, %18\n\t"
      "ds_read_b64_tr_b16 %7, %19\n\t"
      "ds_read_b64_tr_b16 %8, %20\n\t"
      "ds_read_b64_tr_b16 %9, %21\n\t"
      "ds_read_b64_tr_b16 %10, %22\n\t"
      "ds_read_b64_tr_b16 %11, %23\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1]),
        "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
      : "v"(base + koff[0]), "v"(base + koff[1]), "v"(base + koff[2]), "v"(base + koff[3]),
        "v"(base + voff[0]), "v"(base + voff[1]), "v"(base + voff[2]), "v"(base + voff[3]),
        "v"(base + voff[4]), "v"(base + voff[5]), "v"(base + voff[6]), "v"(base + voff[7])
      : "memory");
}
__device__ __forceinline__ void lds_read_k2v4(uint32_t base, const int* koff, const int* voff,
                                              u32x4* k, u32x2* v) {
  asm volatile(
      "ds_read_b128 %0, %6\n\t"
      "ds_read_b128 %1, %7\n\t"
      "ds_read_b64_tr_b16 %2, %8\n\t"
      "ds_read_b64_tr_b16 %3, %9\n\t"
      "ds_read_b64_tr_b16 %4, %10\n\t"
      "ds_read_b64_tr_b16 %5, %11\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(k[0]), "=&v"(k[1]), "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(base + koff[0]), "v"(base + koff[1]), "v"(base + voff[0]), "v"(base + voff[1]),
        "v"(base + voff[2]), "v"(base + voff[3])
      : "memory");
}
template <int D, int WAIT>
__device__ __forceinline__ void lds_read_tile(uint32_t base, const int (&koff)[D / 32],
                                              const int (&voff)[D / 16], u32x4 (&k)[D / 32],
                                              u32x2 (&v)[D / 16]) {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT) : "memory");
  if constexpr (D == 64) {
    lds_read_k2v4(base, koff, voff, k, v);
  } else {
#pragma unroll
    for (int g = 0; g < D / 128; ++g)
      lds_read_k4v8(base, koff + 4 * g, voff + 8 * g, k + 4 * g, v + 8 * g);
  }
}

// Reads the B operand of S^T = K Q^T (query row l16, chunk 4c + grp) from the
// wave's query slot.  The caller has made sure the slot's DMA has landed.
template <int D>
__device__ __forceinline__ void lds_read_q(uint32_t base, const int (&qoff)[D / 32],
                                           u32x4 (&q)[D / 32]) {
#pragma unroll
  for (int c = 0; c < D / 32; c += 2) {
    if constexpr (D / 32 >= 2) {
      asm volatile(
          "ds_read_b128 %0, %2\n\t"
          "ds_read_b128 %1, %3\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(q[c]), "=&v"(q[c + 1])
          : "v"(base + qoff[c]), "v"(base + qoff[c + 1])
          : "memory");
    }
  }
}

template <class T, int D_, int GB>
__global__ __launch_bounds__(DecStream<D_>::kWavesPerWG * 64, DecStream<D_>::kWavesPerSimd)
void decode_stream_kernel(fa_decode_args a, DecodeWsS ws) {
  using S = DecStream<D_>;
  constexpr int D = S::D, TK = S::kTile, PD = S::kDepth, W = S::kWavesPerWG;
  constexpr int RB = S::kRowBytes, RPD = S::kRowsPerDma, LPR = S::kLanesPerRow;
  // Query-slot rows: GB rounded up to whole DMA instructions.
  constexpr int QR = (GB + RPD - 1) / RPD * RPD;
  static_assert(PD >= 2, "at least one tile in flight behind the current one");
  static_assert(GB <= S::kMaxGroup, "query slot holds kMaxGroup rows");
  __shared__ int pfx[S::kMaxBatch + 1];
  __shared__ __attribute__((aligned(16))) char ring[W][PD][S::kTileBytes];
  __shared__ __attribute__((aligned(16))) char qslot[W][QR][RB];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int l16 = lane & 15, grp = lane >> 4;
  const int B = a.batch;
  const int G = a.num_heads / a.num_kv_heads;
  const int ngroups = G / GB;
  const int HG = a.num_kv_heads * ngroups;
  const int cap = a.max_blocks * a.page_size;
  const const_i32_ptr seq_lens = as_const(a.seq_lens);

  // ---- split size, then batch prefix sums of split counts (first wave)
  __shared__ int split_sh;
  if (wv == 0) {
    int split = ws.split;
    int units2 = 0;  // items per head slot at twice the split
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int b = b0 + lane;
      const int len = b < B ? max(0, min(a.seq_lens[b], cap)) : 0;
      units2 += wave_sum_int((len + 2 * split - 1) / (2 * split));
    }
    if ((int64_t)units2 * HG >= (int64_t)tiles::kDecItemsPerWave * gridDim.x * W) split *= 2;
    if (lane == 0) {
      split_sh = split;
      if (blockIdx.x == 0) *ws.split_out = split;
    }
    int base = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int b = b0 + lane;
      int cnt = 0;
      if (b < B) {
        const int len = max(0, min(a.seq_lens[b], cap));
        cnt = (len + split - 1) / split;
      }
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      if (b < B) pfx[b + 1] = base + incl;
      base += __shfl(incl, 63);
    }
    if (lane == 0) pfx[0] = 0;
  }
  __syncthreads();
  const int split = __builtin_amdgcn_readfirstlane(split_sh);
  // Items are numbered unit-major, head-slot-minor.  A workgroup owns a
  // contiguous range of them (a multiple of W long) and wave wv takes every
  // W-th one from offset wv, so at any time the waves of a workgroup work on
  // W consecutive items: with HG = W, the W head slots of one split, whose
  // rows share the cache pages and DRAM rows.
  const int total = __builtin_amdgcn_readfirstlane(pfx[B]) * HG;  // uniform: item state stays scalar
  const int per_wg = (total + gridDim.x * W - 1) / (gridDim.x * W) * W;
  const int I1 = min((int)blockIdx.x * per_wg + per_wg, total);
  const int I0 = blockIdx.x * per_wg + wv;
  if (I0 >= I1) return;

  const float scale_log2 = a.softmax_scale * kLog2e;
  const int ps_log2 = __builtin_ctz(a.page_size);
  const int ps_mask = a.page_size - 1;
  const unsigned last_page = (unsigned)(a.num_pages - 1);
  const int ks1 = (int)a.k_stride[1], vs1 = (int)a.v_stride[1];
  const int64_t ks1b = 2 * (int64_t)ks1, vs1b = 2 * (int64_t)vs1;  // bytes

  // ---- per-lane constants.  DMA: instruction c fills rows RPD c + dl, lane
  // (dl = lane / LPR, pos = lane % LPR) chunk position pos with chunk
  // pos ^ swz(row); offsets in elements from the tile's first row.
  auto swz = [](int r) { return dec_swz(r) & S::kSwzMask; };
  const int dl = lane / LPR, pos = lane % LPR;
  // Head_dim 512 (one wave per SIMD, O in the accumulation registers) has no
  // VGPRs for offset tables: there the offsets below are formed at each use
  // (kBig), the others are tables.
  constexpr bool kBig = D == 512;
  constexpr int NT = kBig ? 1 : S::kDmaPerTensor;
  int kdma[NT], vdma[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) {
    const int r = RPD * c + dl;
    kdma[c] = r * ks1 + 8 * (pos ^ swz(r));
    vdma[c] = r * vs1 + 8 * (pos ^ swz(r));
  }
  // DMA c of a tile (element offsets from its first row).  Head_dim 512: one
  // row per instruction (RPD = 1, dl = 0, pos = lane).
  auto kdma_at = [&](int c) {
    if constexpr (kBig) return c * ks1 + 8 * (lane ^ swz(c)); else return kdma[c];
  };
  auto vdma_at = [&](int c) {
    if constexpr (kBig) return c * vs1 + 8 * (lane ^ swz(c)); else return vdma[c];
  };
  // LDS operand offsets within a ring slot.  K (A operand c of S^T): row l16,
  // chunk 4c + grp.  V^T (A operand of O^T, d block db): lane (k = l16, grp)
  // points at row 4 grp + k / 4, columns 16 db + 4 (k % 4) .. + 3, so that
  // the transpose read hands lane (l16, grp) V[4 grp + j][16 db + l16], j < 4.
  // Head_dim 512: the swizzle acts on the low 4 chunk bits, so chunk 4c + grp
  // of a row lands at 16((4c + grp) ^ sw) = 64(c ^ (sw >> 2)) + 16(grp ^
  // (sw & 3)), i.e. koff(c) = koff(0) ^ 64c; likewise voff(db) = voff(0) ^
  // 32db and qoff(c) = qoff(0) + 64c.
  constexpr int NK = kBig ? 1 : D / 32, NV = kBig ? 1 : D / 16;
  int koff[NK], voff[NV];
#pragma unroll
  for (int c = 0; c < NK; ++c) koff[c] = l16 * RB + 16 * ((4 * c + grp) ^ swz(l16));
  {
    const int r = 4 * grp + (l16 >> 2);
#pragma unroll
    for (int db = 0; db < NV; ++db) {
      const int chunk = 2 * db + ((l16 & 3) >> 1);
      voff[db] = TK * RB + r * RB + 16 * (chunk ^ swz(r)) + 8 * (l16 & 1);
    }
  }
  // Query slot: row h (head h0 + h) holds its RB bytes unswizzled; the B
  // operand c of S^T for column l16 is chunk 4c + grp of row l16 (columns
  // >= GB read row 0 and are zeroed after the read).
  int qoff[NK];
#pragma unroll
  for (int c = 0; c < NK; ++c) qoff[c] = (l16 < GB ? l16 : 0) * RB + 16 * (4 * c + grp);
  const uint32_t ring_base = lds_addr(ring[wv][0]);
  const uint32_t q_base = lds_addr(qslot[wv][0]);

  // ---- producer.  prepare() computes the addresses of tile (pI, pt) and
  // advances to the next tile; issue(slot) then puts its kDmaPerTile DMA
  // instructions (RPD rows each) into ring slot `slot`.  The split lets the
  // address work run before the wait for the tile being replaced, so only
  // the DMA issue separates that tile's arrival from the refill.  Every
  // issue() emits the 8 instructions (after the last tile it reloads that
  // tile), which the fixed vmcnt in lds_read_tile relies on.  The page index
  // of a tile is read (scalar load) one prepare() early.
  int pI = I0, pt = 0;
  DecItem pit = dec_item(pI, pfx, seq_lens, cap, B, HG, ngroups, split);
  bool pdone = false;
  auto page_of = [&](const DecItem& it, int t) -> int {
    const_i32_ptr bt = as_const(a.block_table) + (int64_t)it.b * a.block_table_stride;
    return bt[(it.n_begin + t * TK) >> ps_log2];
  };
  // Pages of fewer than 16 keys (but at least RPD, so that each DMA
  // instruction's RPD rows lie in one page): the page of instruction c's
  // first row (clamped to the tile's last valid row), read in prepare() with
  // a scalar load per instruction and used in issue(), after the tile wait
  // (the loads' latency overlaps it).
  const bool small = a.page_size < TK;
  constexpr int NPG = S::kDmaPerTensor;
  int pgr[NPG];
#pragma unroll
  for (int c = 0; c < NPG; ++c) pgr[c] = 0;
  int page_next = small ? 0 : page_of(pit, 0);
  // Query slot: holds the rows of item q_item (-1: free).  Rows past GB
  // repeat row GB - 1 so that every DMA instruction stays in bounds.
  int q_item = -1;
  // Prepared tile: base rows of K and V, number of valid rows - 1 (15 for a
  // full tile) and the query rows to fetch with it (q_src, or none).
  const uint16_t* kc_n = nullptr;
  const uint16_t* vc_n = nullptr;
  int dr_n = TK - 1;
  const uint16_t* q_src = nullptr;
  int q_h0 = 0;
  auto prepare = [&]() {
    q_src = nullptr;
    if (pt == 0 && q_item < 0 && !pdone) {
      q_src = static_cast<const uint16_t*>(a.q) + (int64_t)pit.b * a.q_stride[0];
      q_h0 = pit.hk * G + pit.hg * GB;
      q_item = pI;
    }
    const int n = pit.n_begin + pt * TK;  // first key of the tile
    dr_n = min(TK - 1, pit.n_end - 1 - n);
    if (small) {
      // Head bases only; the pages are applied per instruction in issue().
      const_i32_ptr bt = as_const(a.block_table) + (int64_t)pit.b * a.block_table_stride;
#pragma unroll
      for (int c = 0; c < NPG; ++c) pgr[c] = bt[(n + min(RPD * c, dr_n)) >> ps_log2];
      kc_n = static_cast<const uint16_t*>(a.k_cache) + (int64_t)pit.hk * a.k_stride[2];
      vc_n = static_cast<const uint16_t*>(a.v_cache) + (int64_t)pit.hk * a.v_stride[2];
    } else {
      const int64_t page = min((unsigned)page_next, last_page);
      const int tok0 = n & ps_mask;  // tiles are 16-aligned and never cross a page
      kc_n = static_cast<const uint16_t*>(a.k_cache) + (int64_t)pit.hk * a.k_stride[2] +
             page * a.k_stride[0] + (int64_t)tok0 * ks1;
      vc_n = static_cast<const uint16_t*>(a.v_cache) + (int64_t)pit.hk * a.v_stride[2] +
             page * a.v_stride[0] + (int64_t)tok0 * vs1;
    }
    if (pdone) return;
    if (pt + 1 < pit.ntiles) {
      ++pt;
    } else if (pI + W < I1) {
      pt = 0;
      pit = dec_item(pI += W, pfx, seq_lens, cap, B, HG, ngroups, split);
    } else {
      pdone = true;  // stays on the last tile
      return;
    }
    if (!small) page_next = page_of(pit, pt);
  };
  auto issue = [&](int slot) {
    if (q_src) {
#pragma unroll
      for (int r0 = 0; r0 < QR; r0 += RPD)
        ld16_lds_nt(q_src + (int64_t)(q_h0 + min(r0 + dl, GB - 1)) * a.q_stride[1] + 8 * pos,
                    qslot[wv][r0]);
    }
    char* kb = ring[wv][slot];
    char* vb = kb + TK * RB;
    if (small) {
      // Instruction c: rows RPD c + dl of one page (the page of its first row
      // clamped to the last valid one, dr_n); rows past dr_n repeat row dr_n.
      // The tile starts a page (16-aligned), so row r sits at slot r & mask.
#pragma unroll
      for (int c = 0; c < S::kDmaPerTensor; ++c) {
        const int r = RPD * c + dl;
        const int64_t page = min((unsigned)pgr[c], last_page);
        const int64_t slot = min(r, dr_n) & ps_mask;
        const int j = 8 * (pos ^ swz(r));
        ld16_lds_nt(kc_n + page * a.k_stride[0] + slot * ks1 + j, kb + 1024 * c);
        ld16_lds_nt(vc_n + page * a.v_stride[0] + slot * vs1 + j, vb + 1024 * c);
      }
    } else if (kBig && dr_n == TK - 1) {
      // Row c at a scalar row pointer stepped by the row stride (opaquely,
      // so that it is not re-derived as a 64-bit product per row) plus the
      // lane's 16-byte chunk, formed per issue from an opaque lane index
      // (not hoisted into a table of addresses across the loop).
      int lb = lane;
      asm volatile("" : "+v"(lb));
      const char* kp = reinterpret_cast<const char*>(kc_n);
      const char* vp = reinterpret_cast<const char*>(vc_n);
#pragma unroll
      for (int c = 0; c < S::kDmaPerTensor; ++c) {
        const uint32_t vo = 16u * (uint32_t)(lb ^ swz(c));
        ld16_lds_nt(kp + vo, kb + 1024 * c);
        ld16_lds_nt(vp + vo, vb + 1024 * c);
        kp += ks1b;
        vp += vs1b;
        asm volatile("" : "+s"(kp), "+s"(vp));
      }
    } else if (dr_n == TK - 1) {
#pragma unroll
      for (int c = 0; c < S::kDmaPerTensor; ++c) {
        ld16_lds_nt(kc_n + kdma_at(c), kb + 1024 * c);
        ld16_lds_nt(vc_n + vdma_at(c), vb + 1024 * c);
      }
    } else {  // last tile of the item: rows past its end repeat the last key
#pragma unroll
      for (int c = 0; c < S::kDmaPerTensor; ++c) {
        const int r = RPD * c + dl;
        const int dr = min(r, dr_n);
        const int j = 8 * (pos ^ swz(r));
        ld16_lds_nt(kc_n + dr * ks1 + j, kb + 1024 * c);
        ld16_lds_nt(vc_n + dr * vs1 + j, vb + 1024 * c);
      }
    }
    // Keeps the next call's DMA behind this one in issue order (the slots are
    // distinct memory, so the compiler could otherwise interleave them).
    asm volatile("" ::: "memory");
  };

  // ---- consumer state.  S^T and O^T use the 16x16x32 layout: lane
  // (l16, grp) holds S^T[key 4 grp + i][head l16] and O^T[16 db + 4 grp + i]
  // [head l16]; ms / lsum belong to head l16.
  int cI = I0, ct = 0;
  DecItem cit = dec_item(cI, pfx, seq_lens, cap, B, HG, ngroups, split);
  u32x4 qb[D / 32];
  float ms = neg_inf(), lsum = 0.f;
  f32x4 o[D / 16];
  auto start_item = [&]() {
    if (q_item == cI) {
      // DMA issued with this item's first tile, before it: resident once
      // that tile has passed its wait.
      if constexpr (kBig) {
        int qo[D / 32];
#pragma unroll
        for (int c = 0; c < D / 32; ++c) qo[c] = qoff[0] + 64 * c;
        lds_read_q<D>(q_base, qo, qb);
      } else {
        lds_read_q<D>(q_base, qoff, qb);
      }
      q_item = -1;
    } else {
      // The slot holds a later item's rows: read this item's rows directly.
      // Only items of a single tile get here.
      const int h0 = cit.hk * G + cit.hg * GB;
      const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + (int64_t)cit.b * a.q_stride[0] +
                             (int64_t)(h0 + min(l16, GB - 1)) * a.q_stride[1];
#pragma unroll
      for (int c = 0; c < D / 32; ++c) qb[c] = ld16(qrow + 32 * c + 8 * grp);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): qb is not left pending
    }
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
      if (l16 >= GB) qb[c] = u32x4{0, 0, 0, 0};  // unused MFMA columns
    ms = neg_inf();
    lsum = 0.f;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto finish_item = [&]() {
    float lt = lsum + __shfl_xor(lsum, 16);
    lt = half_sum(lt);
    if (l16 < GB) {
      const int h = cit.hk * G + cit.hg * GB + l16;
      const int64_t row = ((int64_t)cit.b * a.num_heads + h) * ws.nsplit + cit.c;
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      float* dst = ws.po + row * D + 4 * grp;
#pragma unroll
      for (int db = 0; db < D / 16; ++db)
        *reinterpret_cast<f32x4*>(dst + 16 * db) = o[db] * inv;
      if (grp == 0) ws.plse[row] = lt > 0.f ? ms + log2f(lt) : neg_inf();
    }
  };
  // Consumes the tile held in registers (read out of its ring slot by
  // lds_read_tile, after which the slot is refilled).
  auto consume = [&](const u32x4 (&kr)[D / 32], const u32x2 (&vt)[D / 16]) {
    if (ct == 0) start_item();
    const int n = cit.n_begin + ct * TK;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < D / 32; ++c) s = T::mma16(kr[c], qb[c], s);
    float mt = neg_inf();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (n + 4 * grp + i >= cit.n_end) s[i] = neg_inf();
      mt = fmaxf(mt, s[i]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = half_max(mt) * scale_log2;
    const bool grow = mt > ms + 8.f;
    if (__any(grow)) {
      const float ms_new = grow ? mt : ms;
      const float alpha = grow ? fast_exp2(ms - ms_new) : 1.f;
      ms = ms_new;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) o[db] *= alpha;
    }
    const float mb = ms == neg_inf() ? 0.f : ms;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = fast_exp2(fmaf(s[i], scale_log2, -mb));
      lsum += p[i];
    }
    // B operand of O^T: k slots 8 grp + j hold key 4 grp + j for j < 4 and
    // zero for j >= 4; the A operand repeats its 4 keys in the upper slots.
    if constexpr (kBig) {
      // 16x16x16: the 4 keys of each operand exactly (no duplicated A).
      const u32x2 pb2 = {T::pack(p[0], p[1]), T::pack(p[2], p[3])};
#pragma unroll
      for (int db = 0; db < D / 16; ++db) o[db] = T::mma16k16(vt[db], pb2, o[db]);
    } else {
      const u32x4 pb = {T::pack(p[0], p[1]), T::pack(p[2], p[3]), 0u, 0u};
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        const u32x4 va = {vt[db].x, vt[db].y, vt[db].x, vt[db].y};
        o[db] = T::mma16(va, pb, o[db]);
      }
    }
    if (++ct == cit.ntiles) {
      finish_item();
      ct = 0;
      if ((cI += W) < I1) cit = dec_item(cI, pfx, seq_lens, cap, B, HG, ngroups, split);
    }
  };

  // ---- pipeline: a step prepares the tile PD ahead, reads the tile in ring
  // slot s into registers, refills the slot and then computes, so PD tiles
  // are in flight during the compute.  The loop leaves only after a whole
  // group of PD steps; loads past the last tile only reload it.
#pragma unroll
  for (int s = 0; s < PD; ++s) {
    prepare();
    issue(s);
  }
  do {
#pragma unroll
    for (int s = 0; s < PD; ++s) {
      u32x4 kr[D / 32];
      u32x2 vt[D / 16];
      prepare();
      // Pins the prepared addresses ahead of the wait (volatile asm keeps its
      // order; the compiler would otherwise sink the address work past it).
      asm volatile("" ::"s"(kc_n), "s"(vc_n), "s"(dr_n), "s"(q_src));
      if constexpr (kBig) {
        // Offsets formed here (opaquely rewritten bases: not hoisted into
        // tables across the loop).
        int kb0 = koff[0], vb0 = voff[0];
        asm volatile("" : "+v"(kb0), "+v"(vb0));
        int ko[D / 32], vo[D / 16];
#pragma unroll
        for (int c = 0; c < D / 32; ++c) ko[c] = kb0 ^ (64 * c);
#pragma unroll
        for (int db = 0; db < D / 16; ++db) vo[db] = vb0 ^ (32 * db);
        lds_read_tile<D, (PD - 1) * S::kDmaPerTile>(ring_base + s * S::kTileBytes, ko, vo, kr,
                                                    vt);
      } else {
        lds_read_tile<D, (PD - 1) * S::kDmaPerTile>(ring_base + s * S::kTileBytes, koff, voff,
                                                    kr, vt);
      }
      issue(s);
      if (cI < I1) consume(kr, vt);
    }
  } while (cI < I1);
  // No DMA may still be writing this wave's LDS when the wave ends.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
}

}  // namespace fa
