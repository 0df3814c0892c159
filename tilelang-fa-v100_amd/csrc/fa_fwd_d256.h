// Attention forward core for head_dim 256 on gfx950 (dense rows, and paged
// rows with pages of at least 16 keys): 4 waves x 32 query rows (128 rows
// per workgroup), one wave per SIMD, 32-key tiles.
//  * O (32 rows x 256 d, 128 registers) lives in AGPRs for the whole tile
//    (mma32_agpr), Q (64) and the scores in VGPRs: one pass over the keys
//    with 512 registers per wave.  (Two waves per SIMD would need O in two
//    128-column passes with the scores recomputed, 1.5x the products.)
//  * Software pipeline inside the wave, which issues in order and has no
//    partner wave on its SIMD: iteration j computes Sᵀ(j + 1) while tile j
//    is exponentiated, then Oᵀ += Vᵀ(j) Pᵀ(j) while tile j + 1's row max and
//    rescale decision are taken.  The softmax work is cut into slices with
//    no dependence between neighbouring slices, one slice per product, so
//    the next product issues while the previous one runs.
//  * K and V tiles are 32 rows of 512 bytes; 16-byte chunk q of row r is
//    stored at chunk q ^ swz(r), the XOR touching the low four chunk bits
//    (chunks stay in their 256-byte half).  Each wave DMAs 8 rows of each
//    (four 1 KB blocks) through a buffer resource, one block every four
//    products of a chain: K(j + 2) during Sᵀ(j + 1) (K double buffered),
//    V(j + 2) during Oᵀ(j) (V triple buffered, so it has a tile and a half
//    to land).
#pragma once

#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

struct FwdShapeD256 {
  static constexpr int D = 256;
  static constexpr int BM = tiles::kFwd256Rows;  // 4 waves x 32 rows
  static constexpr int BN = 32;
  static constexpr int NW = 4;
  static constexpr int ROWB = 2 * D;         // bytes per K / V row
  static constexpr int TILEB = BN * ROWB;    // 16 KB
  static_assert(BM == 32 * NW, "one 32-row block per wave");
};

// smem: 5 TILEB bytes of LDS: two K tiles, then three V tiles (picked at run
// time: 16 KB offsets leave the XOR-combined bits of the operand offsets
// alone).  K first, so K operand offsets stay instruction immediates.
template <class T, class Prob>
__device__ __forceinline__ void attn_fwd_tile_d256(const Prob& P, int row0, float scale,
                                                   char* smem) {
  char* const k0 = smem;
  char* const k1 = smem + FwdShapeD256::TILEB;
  char* const vbuf = smem + 2 * FwdShapeD256::TILEB;
  using S = FwdShapeD256;
  constexpr int D = S::D, BN = S::BN;
  const float scale_log2 = scale * kLog2e;
  constexpr float kLazy = 8.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;

  const int nrows = P.nrows;
  const int row_last = min(row0 + S::BM, nrows) - 1;
  const int wg_lo = P.kv_lo(row0);
  const int wg_hi = P.kv_hi(row_last);

  const int wrow0 = row0 + wave * 32;
  const bool wave_active = wrow0 < nrows;
  const int wrow_last = min(wrow0 + 31, nrows - 1);
  const int w_lo_min = wave_active ? P.kv_lo(wrow0) : 0;
  const int w_lo_max = wave_active ? P.kv_lo(wrow_last) : 0;
  const int w_hi_min = wave_active ? P.kv_hi(wrow0) : 0;
  const int w_hi_max = wave_active ? P.kv_hi(wrow_last) : 0;

  const int row = wrow0 + lr;
  const bool row_valid = row < nrows;
  const int my_lo = row_valid ? P.kv_lo(row) : 0;
  const int my_hi = row_valid ? P.kv_hi(row) : 0;

  u32x4 qf[D / 16];
  {
    const uint16_t* qp = row_valid ? P.q_ptr(row) : nullptr;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      qf[c] = row_valid ? ld16(qp + 16 * c + 8 * lh) : u32x4{0, 0, 0, 0};
  }

  // Sᵀ operand of step c: row lr, logical chunk 2c + lh, stored at
  // (2c + lh) ^ swz(lr) within its 256-byte half, i.e. byte offset
  // kbase ^ 32c (bit 8 of 32c selects the half).  Vᵀ operand, 16-key chunk kc, d tile dt: lane k reads row 16kc +
  // 4(k/32) + (k%16)/4 (+8 for the upper half), logical chunk 4dt + q with
  // q = 2((k/16)%2) + (k%4)/2; stored at (4dt + q) ^ swz(row), i.e. byte
  // offset vbase[hf] ^ 64dt.
  int kbase = lr * S::ROWB + 16 * (lh ^ swz_chunk(lr));
  int vbase[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * hf;
    const int q = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int sw = swz_chunk(r);
    vbase[hf] = r * S::ROWB + 64 * (sw >> 2) + 16 * (q ^ (sw & 3)) + 8 * (lane & 1);
  }

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
    agpr_fence_in(o[dt]);
  }
  float ms_run = neg_inf(), l_run = 0.f;
  bool o_live = false;  // wave-uniform: an O product has been issued
  u32x4 pb[BN / 16];
  constexpr int kAheadS = FA_FWD_AHEAD_S, kAheadO = FA_FWD_AHEAD_O;

  auto visible = [&](int j) {
    return wave_active && j * BN < w_hi_max && j * BN + BN > w_lo_min;
  };
  // acc = K Qᵀ for the tile in kb; extra(c) runs after the product of step c.
  auto gemm_s = [&](f32x16& acc, const char* kb, auto extra) {
    asm volatile("" : "+v"(kbase));
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    lds_pipeline<D / 16, kAheadS>(
        [&](int c) { return ld16(kb + (kbase ^ (32 * c))); },
        [&](int c, const u32x4& k) {
          acc = T::mma32(k, qf[c], acc);
          extra(c);
        });
  };
  // O += Vᵀ Pᵀ for the V tile at byte offset voff of vbuf; extra(k) runs
  // after the product of step k.
  auto gemm_o = [&](int voff, auto extra) {
    const int vb0 = vbase[0] + voff, vb1 = vbase[1] + voff;  // XOR bits untouched
    struct VOps {
      u32x2 lo, hi;
    };
    lds_pipeline<(BN / 16) * (D / 32), kAheadO>(
        [&](int k) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          const int ro = kc * 16 * S::ROWB;
          return VOps{lds_read_tr(vbuf + (vb0 ^ (64 * dt)) + ro),
                      lds_read_tr(vbuf + (vb1 ^ (64 * dt)) + ro)};
        },
        [&](int k, const VOps& r) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          mma32_agpr<T>(o[dt], u32x4{r.lo[0], r.lo[1], r.hi[0], r.hi[1]}, pb[kc]);
          extra(k);
        });
  };

  // ---- DMA: wave w fills rows 8w .. 8w + 7 of a K or V tile (blocks
  // 4w .. 4w + 3, two rows per 1 KB block) through a buffer resource; lane
  // offsets are fixed, rows at or past wg_hi read as zero.  A tile's DMA is
  // issued in pieces spread over a matrix chain (the resource, then one
  // block every four products): the CU's vector-memory path takes tens of
  // cycles per 1 KB block, and four waves issuing all their blocks at once
  // left the matrix cores idle for ~400 cycles per tile.
  uint32_t k_loff[4], v_loff[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int r8 = 2 * ii + (lane >> 5);
    const uint32_t c = (lane & 31) ^ swz_chunk(8 * wave + r8);
    k_loff[ii] = 2u * ((uint32_t)r8 * (uint32_t)P.k_row_stride() + 8u * c);
    v_loff[ii] = 2u * ((uint32_t)r8 * (uint32_t)P.v_row_stride() + 8u * c);
  }
  const int j0 = max(wg_lo, 0) / BN;
  const int j1 = (wg_hi + BN - 1) / BN;
  // Tiles are requested in increasing order, K and V each, also past the
  // last tile (a zero-byte resource: nothing is read, zeros land in a free
  // buffer).  Row-strided problems step a per-wave row pointer by one tile
  // per request instead of a 64-bit row product; paged problems resolve the
  // row through the block table, at the last visible row for tiles past the
  // end (only entries of the sequence's pages are read).
  const uint16_t* k_next = nullptr;
  const uint16_t* v_next = nullptr;
  if constexpr (Prob::kRowStrided) {
    k_next = P.k_ptr(j0 * BN + 8 * wave);
    v_next = P.v_ptr(j0 * BN + 8 * wave);
  }
  auto dma_rsrc = [&](int n0, auto is_v) {
    constexpr bool kV = decltype(is_v)::value;
    const int nw = n0 + 8 * wave;
    const int nvalid = min(8, wg_hi - nw);
    const uint16_t* base;
    if constexpr (Prob::kRowStrided) {
      const uint16_t*& cur = kV ? v_next : k_next;
      base = cur;
      cur += BN * (kV ? P.v_row_stride() : P.k_row_stride());
    } else {
      const int nb = nvalid > 0 ? nw : wg_hi - 1;
      base = kV ? P.v_ptr(nb) : P.k_ptr(nb);
    }
    const uint32_t bytes = span_bytes(nvalid, kV ? P.v_row_stride() : P.k_row_stride(), D);
    u32x4 rs = rsrc_words(base, bytes);
#pragma unroll
    for (int w = 0; w < 4; ++w) rs[w] = __builtin_amdgcn_readfirstlane(rs[w]);
    return rs;
  };
  auto dma_block = [&](const u32x4& rs, char* dst, int ii, auto is_v) {
    constexpr bool kV = decltype(is_v)::value;
    buffer_lds16_opaque(rs, kV ? v_loff[ii] : k_loff[ii], dst + (4 * wave + ii) * 1024);
  };
  // The whole DMA of one tile at once (prologue, and steps without a chain).
  auto dma_tile = [&](int n0, char* dst, auto is_v) {
    const u32x4 rs = dma_rsrc(n0, is_v);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) dma_block(rs, dst, ii, is_v);
  };

  // ---- Online softmax of a tile in two stages that ride on the matrix
  // chains.  Stage A (mask, row max, rescale decision) of tile t runs in the
  // O chain of tile t - 1; stage B (P = exp2(S·scale − max), packed into pb
  // and summed into l_run) in the S chain of tile t + 1.  Both are sliced so
  // that no slice waits for the previous one's result.
  // Each slice's result is pinned to its slot (an empty asm that takes it as
  // an operand): otherwise the compiler sinks the slices next to their first
  // use, out of the chain.
  auto pin = [](float& x) { asm volatile("" : "+v"(x)); };
  float alpha = 1.f, mb = 0.f;  // tile t's rescale factor and exponent offset
  bool grow = false;
  float mt = neg_inf();
  auto mask_tile = [&](f32x16& sc, int n0) {
    if ((n0 < w_lo_max) || (n0 + BN > w_hi_min)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kv = n0 + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (kv < my_lo || kv >= my_hi) sc[i] = neg_inf();
      }
    }
  };
  // Slices 0-5 at O-chain steps 1, 3, .., 11.  live: the tile is visible to
  // the wave (otherwise its scores are stale and nothing may change).
  auto stage_a = [&](const f32x16& sc, int k, bool live) {
    if (k & 1 || k > 11) return;
    const int a = k >> 1;
    if (a == 0) {
      mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      pin(mt);
    } else if (a < 4) {
#pragma unroll
      for (int i = 4 * a; i < 4 * a + 4; ++i) mt = fmaxf(mt, sc[i]);
      pin(mt);
    } else if (a == 4) {
      mt = half_max(mt) * scale_log2;
      pin(mt);
    } else {
      // A row's max only moves when the tile max exceeds it by more than
      // kLazy, so P <= 2^kLazy and O is rescaled on few tiles.
      grow = live && mt > ms_run + kLazy;
      const float ms_new = grow ? mt : ms_run;
      alpha = grow ? fast_exp2(ms_run - ms_new) : 1.f;
      ms_run = ms_new;
      l_run *= alpha;
      // A row with no visible key so far has ms_run = -inf and only -inf
      // scores in this tile: any finite offset gives P = 0.
      mb = ms_run == neg_inf() ? 0.f : ms_run;
      pin(mb);
      pin(l_run);
    }
  };
  // Step c (0..17): exponent argument of element c, exponential of element
  // c - 1, pack and sum (into lt) of the pair whose second exponential ran
  // at c - 1.
  auto stage_b = [&](f32x16& sc, int c, float& lt) {
    if (c < 16) {
      float x = fmaf(sc[c], scale_log2, -mb);
      pin(x);
      sc[c] = x;
    }
    if (c >= 1 && c <= 16) {
      float x = fast_exp2(sc[c - 1]);
      pin(x);
      sc[c - 1] = x;
    }
    if (c >= 3 && (c & 1)) {
      const int pr = (c - 3) >> 1, e = 2 * pr;
      uint32_t w = T::pack(sc[e], sc[e + 1]);
      asm volatile("" : "+v"(w));
      pb[pr >> 2][pr & 3] = w;
      lt = T::sum2(sc[e], sc[e + 1], w, lt);
      pin(lt);
    }
  };
  auto tile_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  auto rescale_o = [&]() {
    if (o_live && __any(grow)) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        agpr_fence_out(o[dt]);
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
      }
    }
  };

  // ---- Step j (after the barrier: K(j + 1) and V(j) resident, every wave
  // done with tile j - 1's buffers): Sᵀ(j + 1) = K(j + 1) Qᵀ with stage B of
  // tile j and the DMA of K(j + 2) into kd; stage A of tile j + 1 inside
  // O += Vᵀ(j) Pᵀ(j), with the DMA of V(j + 2) into vd.  K is double
  // buffered, V triple buffered (its DMA is issued late in the step).  cur
  // holds tile j's scores, nxt receives tile j + 1's.
  auto step = [&](int j, const char* kn, char* kd, int vc, int vd, f32x16& cur, f32x16& nxt) {
    // K(j + 1) and V(j) must have landed; V(j + 1), each wave's newest DMA,
    // may still be in flight (vmcnt completes in order).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    const bool vis = visible(j);
    const bool vis_n = j + 1 < j1 && visible(j + 1);
    u32x4 rk, rv;
    auto k_piece = [&](int c) {
      if (c == 0) rk = dma_rsrc((j + 2) * BN, BoolC<false>{});
      if ((c & 3) == 2) dma_block(rk, kd, c >> 2, BoolC<false>{});
    };
    auto v_piece = [&](int k) {
      if (k == 0) rv = dma_rsrc((j + 2) * BN, BoolC<true>{});
      if ((k & 3) == 2) dma_block(rv, vbuf + vd, k >> 2, BoolC<true>{});
    };
    // One copy of each chain: stage B of tile j rides on the S chain even
    // when tile j is not visible (its sum is then dropped), stage A of tile
    // j + 1 on the O chain even when tile j + 1 is not (no rescale then).
    // The S chain runs on every step (past a wave's last visible tile it
    // scores whatever K buffer holds, finite data, and the result is never
    // used): a second, chain-less copy of stage B would let the compiler
    // hoist the slices common to both copies out of the chain.
    float lt = l_run;
    gemm_s(nxt, kn, [&](int c) {
      stage_b(cur, c, lt);
      k_piece(c);
    });
    if (vis_n) mask_tile(nxt, (j + 1) * BN);
    stage_b(cur, 16, lt);
    stage_b(cur, 17, lt);
    if (vis) {
      l_run = lt;
      rescale_o();  // tile j's factor, decided in stage A (previous step)
      gemm_o(vc, [&](int k) {
        stage_a(nxt, k, vis_n);
        v_piece(k);
      });
      o_live = true;
    } else {
      dma_tile((j + 2) * BN, vbuf + vd, BoolC<true>{});
#pragma unroll
      for (int k = 0; k < 12; ++k) stage_a(nxt, k, vis_n);
    }
  };

  if (j0 < j1) {
    f32x16 sa, sb;
    dma_tile(j0 * BN, k0, BoolC<false>{});
    tile_barrier();
    dma_tile((j0 + 1) * BN, k1, BoolC<false>{});
    dma_tile(j0 * BN, vbuf, BoolC<true>{});
    dma_tile((j0 + 1) * BN, vbuf + S::TILEB, BoolC<true>{});
    if (visible(j0)) {
      gemm_s(sa, k0, [](int) {});
      mask_tile(sa, j0 * BN);
#pragma unroll
      for (int k = 0; k < 12; ++k) stage_a(sa, k, true);
    }
    // K(t) in buffer t mod 2 and V(t) in buffer t mod 3 (t relative to j0):
    // vc, vd are the byte offsets of V(j) and of V(j + 2).
    constexpr int TB = S::TILEB;
    int vc = 0, vd = 2 * TB;
    auto rot = [](int x) { return x == 2 * TB ? 0 : x + TB; };
    for (int j = j0;; j += 2) {
      step(j, k1, k0, vc, vd, sa, sb);
      if (j + 1 >= j1) break;
      vc = rot(vc);
      vd = rot(vd);
      step(j + 1, k0, k1, vc, vd, sb, sa);
      if (j + 2 >= j1) break;
      vc = rot(vc);
      vd = rot(vd);
    }
    wait_vmem();  // the DMAs requested past the last tile
  }

#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) agpr_fence_out(o[dt]);
  const float l_all = half_sum(l_run);
  if (row_valid) fwd_store_row<T>(P, row, lh, o, l_all, ms_run);
}

}  // namespace fa
