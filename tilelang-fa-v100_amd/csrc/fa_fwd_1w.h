// Attention forward core with one wave per SIMD (gfx950), used for head_dim
// 256 (dense rows, and paged rows with pages of at least 16 keys): 4 waves
// x 32 query rows per workgroup, 32-key tiles.  RB (row blocks of 32 rows
// per wave, each K / V operand read feeding RB products) is 1 here; RB = 2
// at head_dim 128 compiled without spills but ran slower than the two-wave
// ping-pong core (a lone wave issues at most one instruction per four-cycle
// slot, and this loop issues ~300 instructions per 32 products).
//  * O (RB x 32 rows x D, 128 registers) lives in AGPRs for the whole tile
//    (mma32_agpr), Q and the scores in VGPRs: one pass over the keys with 512
//    registers per wave.
//  * Software pipeline inside the wave, which issues in order and has no
//    partner wave on its SIMD: iteration j computes Sᵀ(j + 1) while tile j
//    is exponentiated, then Oᵀ += Vᵀ(j) Pᵀ(j) while tile j + 1's row max and
//    rescale decision are taken.  The softmax work is cut into slices with
//    no dependence between neighbouring slices, spread over the products,
//    so the next product issues while the previous one runs.
//  * K and V tiles are 32 rows of 2D bytes; 16-byte chunk q of row r is
//    stored at chunk q ^ swz(r), the XOR touching the low four chunk bits
//    (chunks stay in their 256-byte half).  Each wave DMAs 8 rows of each
//    through a buffer resource, one 1 KB block every four products of a
//    chain: K(j + 2) during Sᵀ(j + 1) (K double buffered), V(j + 2) during
//    Oᵀ(j) (V triple buffered, so it has a tile and a half to land).
#pragma once

#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

template <int D_, int RB_>
struct FwdShape1W {
  static constexpr int D = D_;
  static constexpr int RB = RB_;               // 32-row blocks per wave
  static constexpr int NW = 4;                 // waves, one per SIMD
  static constexpr int BM = 32 * RB * NW;      // query rows per workgroup
  static constexpr int BN = 32;                // keys per tile
  static constexpr int ROWB = 2 * D;           // bytes per K / V row
  static constexpr int TILEB = BN * ROWB;      // 8 or 16 KB
  static constexpr int KSTEPS = D / 16;        // products per row block in Sᵀ
  static constexpr int OSTEPS = (BN / 16) * (D / 32);  // and in Oᵀ
  static constexpr int RPB = 1024 / ROWB;      // rows per 1 KB DMA block
  static constexpr int CPR = D / 8;            // 16-byte chunks per row
  static constexpr int BPW = 8 / RPB;          // DMA blocks per wave and tile
  static_assert(D == 256 && RB == 1, "instance in use (see the header)");
  static_assert(KSTEPS >= 8 && OSTEPS >= 8 && BPW <= 4, "slice placement");
};

// smem: 5 TILEB bytes of LDS: two K tiles, then three V tiles (picked at run
// time: TILEB offsets leave the XOR-combined bits of the operand offsets
// alone).  K first, so K operand offsets stay instruction immediates.
template <class T, int D_, int RB_, class Prob>
__device__ __forceinline__ void attn_fwd_tile_1w(const Prob& P, int row0, float scale,
                                                 char* smem) {
  using S = FwdShape1W<D_, RB_>;
  constexpr int D = S::D, RB = S::RB, BN = S::BN;
  char* const k0 = smem;
  char* const k1 = smem + S::TILEB;
  char* const vbuf = smem + 2 * S::TILEB;
  const float scale_log2 = scale * kLog2e;
  constexpr float kLazy = 8.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;

  const int nrows = P.nrows;
  const int row_last = min(row0 + S::BM, nrows) - 1;
  const int wg_lo = P.kv_lo(row0);
  const int wg_hi = P.kv_hi(row_last);

  // The wave's rows wrow0 .. wrow0 + 32 RB - 1; row block rb, lane (lr, lh):
  // row wrow0 + 32 rb + lr.
  const int wrow0 = row0 + wave * 32 * RB;
  const bool wave_active = wrow0 < nrows;
  const int wrow_last = min(wrow0 + 32 * RB - 1, nrows - 1);
  const int w_lo_min = wave_active ? P.kv_lo(wrow0) : 0;
  const int w_lo_max = wave_active ? P.kv_lo(wrow_last) : 0;
  const int w_hi_min = wave_active ? P.kv_hi(wrow0) : 0;
  const int w_hi_max = wave_active ? P.kv_hi(wrow_last) : 0;

  int my_lo[RB], my_hi[RB];
  u32x4 qf[RB][D / 16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = wrow0 + 32 * rb + lr;
    const bool row_valid = row < nrows;
    my_lo[rb] = row_valid ? P.kv_lo(row) : 0;
    my_hi[rb] = row_valid ? P.kv_hi(row) : 0;
    const uint16_t* qp = row_valid ? P.q_ptr(row) : nullptr;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      qf[rb][c] = row_valid ? ld16(qp + 16 * c + 8 * lh) : u32x4{0, 0, 0, 0};
  }

  // Sᵀ operand of step c: row lr, logical chunk 2c + lh, stored at
  // (2c + lh) ^ swz(lr) within its 256-byte half, i.e. byte offset
  // kbase ^ 32c (bit 8 of 32c selects the half).  Vᵀ operand, 16-key chunk
  // kc, d tile dt: lane k reads row 16kc + 4(k/32) + (k%16)/4 (+8 for the
  // upper half), logical chunk 4dt + q with q = 2((k/16)%2) + (k%4)/2;
  // stored at (4dt + q) ^ swz(row), i.e. byte offset vbase[hf] ^ 64dt.
  int kbase = lr * S::ROWB + 16 * (lh ^ swz_chunk(lr));
  int vbase[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * hf;
    const int q = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int sw = swz_chunk(r);
    vbase[hf] = r * S::ROWB + 64 * (sw >> 2) + 16 * (q ^ (sw & 3)) + 8 * (lane & 1);
  }

  f32x16 o[RB][D / 32];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) o[rb][dt][i] = 0.f;
      agpr_fence_in(o[rb][dt]);
    }
  float ms_run[RB], l_run[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    ms_run[rb] = neg_inf();
    l_run[rb] = 0.f;
  }
  bool o_live = false;  // wave-uniform: an O product has been issued
  u32x4 pb[RB][BN / 16];
  constexpr int kAheadS = FA_FWD_AHEAD_S, kAheadO = FA_FWD_AHEAD_O;

  auto visible = [&](int j) {
    return wave_active && j * BN < w_hi_max && j * BN + BN > w_lo_min;
  };
  // acc = K Qᵀ for the tile in kb (one operand read, RB products per step);
  // extra(c) runs after the products of step c.
  auto gemm_s = [&](f32x16 (&acc)[RB], const char* kb, auto extra) {
    asm volatile("" : "+v"(kbase));
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][i] = 0.f;
    lds_pipeline<S::KSTEPS, kAheadS>(
        [&](int c) { return ld16(kb + (kbase ^ (32 * c))); },
        [&](int c, const u32x4& k) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) acc[rb] = T::mma32(k, qf[rb][c], acc[rb]);
          extra(c);
        });
  };
  // O += Vᵀ Pᵀ for the V tile at byte offset voff of vbuf; extra(k) runs
  // after the products of step k.
  auto gemm_o = [&](int voff, auto extra) {
    const int vb0 = vbase[0] + voff, vb1 = vbase[1] + voff;  // XOR bits untouched
    struct VOps {
      u32x2 lo, hi;
    };
    lds_pipeline<S::OSTEPS, kAheadO>(
        [&](int k) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          const int ro = kc * 16 * S::ROWB;
          return VOps{lds_read_tr(vbuf + (vb0 ^ (64 * dt)) + ro),
                      lds_read_tr(vbuf + (vb1 ^ (64 * dt)) + ro)};
        },
        [&](int k, const VOps& r) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          const u32x4 a = {r.lo[0], r.lo[1], r.hi[0], r.hi[1]};
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) mma32_agpr<T>(o[rb][dt], a, pb[rb][kc]);
          extra(k);
        });
  };

  // ---- DMA: wave w fills rows 8w .. 8w + 7 of a K or V tile (1 KB blocks
  // BPW w .. BPW w + BPW - 1, RPB rows each) through a buffer resource; lane
  // offsets are fixed, rows at or past wg_hi read as zero.  A tile's DMA is
  // issued in pieces spread over a matrix chain (the resource, then one
  // block every four products): the CU's vector-memory path takes tens of
  // cycles per 1 KB block, and four waves issuing all their blocks at once
  // left the matrix cores idle for ~400 cycles per tile.
  uint32_t k_loff[S::BPW], v_loff[S::BPW];
#pragma unroll
  for (int ii = 0; ii < S::BPW; ++ii) {
    const int r8 = S::RPB * ii + lane / S::CPR;
    const uint32_t c = (lane % S::CPR) ^ swz_chunk(8 * wave + r8);
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
    buffer_lds16_opaque(rs, kV ? v_loff[ii] : k_loff[ii], dst + (S::BPW * wave + ii) * 1024);
  };
  // The whole DMA of one tile at once (prologue, and steps without a chain).
  auto dma_tile = [&](int n0, char* dst, auto is_v) {
    const u32x4 rs = dma_rsrc(n0, is_v);
#pragma unroll
    for (int ii = 0; ii < S::BPW; ++ii) dma_block(rs, dst, ii, is_v);
  };
  // Piece c of a chain: the resource at step 0, block ii at step 4 ii + 2.
  auto dma_piece = [&](int c, u32x4& rs, int n0, char* dst, auto is_v) {
    if (c == 0) rs = dma_rsrc(n0, is_v);
    if ((c & 3) == 2 && (c >> 2) < S::BPW) dma_block(rs, dst, c >> 2, is_v);
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
  float alpha[RB], mb[RB], mt[RB];  // tile t's rescale factor, exponent offset, row max
  bool grow = false;                // some row of the wave rescales
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    alpha[rb] = 1.f;
    mb[rb] = 0.f;
    mt[rb] = neg_inf();
  }
  auto mask_tile = [&](f32x16 (&sc)[RB], int n0) {
    if ((n0 < w_lo_max) || (n0 + BN > w_hi_min)) {
      // Keeps this a branch: if-converted, the selects ran on every tile.
      asm volatile("");
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = n0 + 8 * (i >> 2) + 4 * lh + (i & 3);
          if (kv < my_lo[rb] || kv >= my_hi[rb]) sc[rb][i] = neg_inf();
        }
    }
  };
  // Slice a (0..5) at O-chain step k = AS a + AS - 1.  live: the tile is
  // visible to the wave (otherwise its scores are stale and nothing may
  // change).
  constexpr int AS = S::OSTEPS / 8;
  auto stage_a = [&](const f32x16 (&sc)[RB], int k, bool live) {
    if (k % AS != AS - 1 || k / AS > 5) return;
    const int a = k / AS;
    bool g = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (a == 0) {
        mt[rb] = fmaxf(fmaxf(sc[rb][0], sc[rb][1]), fmaxf(sc[rb][2], sc[rb][3]));
        pin(mt[rb]);
      } else if (a < 4) {
#pragma unroll
        for (int i = 4 * a; i < 4 * a + 4; ++i) mt[rb] = fmaxf(mt[rb], sc[rb][i]);
        pin(mt[rb]);
      } else if (a == 4) {
        mt[rb] = half_max(mt[rb]) * scale_log2;
        pin(mt[rb]);
      } else {
        // A row's max only moves when the tile max exceeds it by more than
        // kLazy, so P <= 2^kLazy and O is rescaled on few tiles.
        const bool gr = live && mt[rb] > ms_run[rb] + kLazy;
        const float ms_new = gr ? mt[rb] : ms_run[rb];
        alpha[rb] = gr ? fast_exp2(ms_run[rb] - ms_new) : 1.f;
        ms_run[rb] = ms_new;
        l_run[rb] *= alpha[rb];
        // A row with no visible key so far has ms_run = -inf and only -inf
        // scores in this tile: any finite offset gives P = 0.
        mb[rb] = ms_run[rb] == neg_inf() ? 0.f : ms_run[rb];
        pin(mb[rb]);
        pin(l_run[rb]);
        g = g || gr;
      }
    }
    if (a == 5) grow = g;
  };
  // Micro-step c (0..17) of row block rb: exponent argument of element c,
  // exponential of element c - 1, pack and sum (into lt) of the pair whose
  // second exponential ran at c - 1.  MPS micro-steps ride on each S-chain
  // step, the last ones follow the chain.
  constexpr int MPS = 16 / S::KSTEPS;
  auto stage_b = [&](f32x16 (&sc)[RB], int c, float (&lt)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (c < 16) {
        float x = fmaf(sc[rb][c], scale_log2, -mb[rb]);
        pin(x);
        sc[rb][c] = x;
      }
      if (c >= 1 && c <= 16) {
        float x = fast_exp2(sc[rb][c - 1]);
        pin(x);
        sc[rb][c - 1] = x;
      }
      if (c >= 3 && (c & 1)) {
        const int pr = (c - 3) >> 1, e = 2 * pr;
        uint32_t w = T::pack(sc[rb][e], sc[rb][e + 1]);
        asm volatile("" : "+v"(w));
        pb[rb][pr >> 2][pr & 3] = w;
        lt[rb] = T::sum2(sc[rb][e], sc[rb][e + 1], w, lt[rb]);
        pin(lt[rb]);
      }
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
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          agpr_fence_out(o[rb][dt]);
#pragma unroll
          for (int i = 0; i < 16; ++i) o[rb][dt][i] *= alpha[rb];
        }
    }
  };

  // ---- Step j (after the barrier: K(j + 1) and V(j) resident, every wave
  // done with tile j - 1's buffers): Sᵀ(j + 1) = K(j + 1) Qᵀ with stage B of
  // tile j and the DMA of K(j + 2) into kd; stage A of tile j + 1 inside
  // O += Vᵀ(j) Pᵀ(j), with the DMA of V(j + 2) into vd.  cur holds tile j's
  // scores, nxt receives tile j + 1's.
  auto step = [&](int j, const char* kn, char* kd, int vc, int vd, f32x16 (&cur)[RB],
                  f32x16 (&nxt)[RB]) {
    // K(j + 1) and V(j) must have landed; V(j + 1), each wave's newest DMA
    // (BPW blocks), may still be in flight (vmcnt completes in order).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70 | S::BPW);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    const bool vis = visible(j);
    const bool vis_n = j + 1 < j1 && visible(j + 1);
    u32x4 rk, rv;
    // One copy of each chain: stage B of tile j rides on the S chain even
    // when tile j is not visible (its sum is then dropped), stage A of tile
    // j + 1 on the O chain even when tile j + 1 is not (no rescale then).
    // The S chain runs on every step (past a wave's last visible tile it
    // scores whatever K buffer holds, finite data, and the result is never
    // used): a second, chain-less copy of stage B would let the compiler
    // hoist the slices common to both copies out of the chain.
    float lt[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) lt[rb] = l_run[rb];
    gemm_s(nxt, kn, [&](int c) {
#pragma unroll
      for (int m = 0; m < MPS; ++m) stage_b(cur, MPS * c + m, lt);
      dma_piece(c, rk, (j + 2) * BN, kd, BoolC<false>{});
    });
    if (vis_n) mask_tile(nxt, (j + 1) * BN);
    stage_b(cur, 16, lt);
    stage_b(cur, 17, lt);
    if (vis) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) l_run[rb] = lt[rb];
      rescale_o();  // tile j's factor, decided in stage A (previous step)
      gemm_o(vc, [&](int k) {
        stage_a(nxt, k, vis_n);
        dma_piece(k, rv, (j + 2) * BN, vbuf + vd, BoolC<true>{});
      });
      o_live = true;
    } else {
      dma_tile((j + 2) * BN, vbuf + vd, BoolC<true>{});
#pragma unroll
      for (int k = 0; k < S::OSTEPS; ++k) stage_a(nxt, k, vis_n);
    }
  };

  if (j0 < j1) {
    f32x16 sa[RB], sb[RB];
    dma_tile(j0 * BN, k0, BoolC<false>{});
    tile_barrier();
    dma_tile((j0 + 1) * BN, k1, BoolC<false>{});
    dma_tile(j0 * BN, vbuf, BoolC<true>{});
    dma_tile((j0 + 1) * BN, vbuf + S::TILEB, BoolC<true>{});
    if (visible(j0)) {
      gemm_s(sa, k0, [](int) {});
      mask_tile(sa, j0 * BN);
#pragma unroll
      for (int k = 0; k < S::OSTEPS; ++k) stage_a(sa, k, true);
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
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) agpr_fence_out(o[rb][dt]);
    const int row = wrow0 + 32 * rb + lr;
    const float l_all = half_sum(l_run[rb]);
    if (row < nrows) fwd_store_row<T>(P, row, lh, o[rb], l_all, ms_run[rb]);
  }
}

}  // namespace fa
