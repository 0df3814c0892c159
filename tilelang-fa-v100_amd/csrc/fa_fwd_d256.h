// Attention forward core for head_dim 256 on gfx950: the two-phase
// (ping-pong) schedule of attn_fwd_tile_d128 with the operands resized.
//
//  * 8 waves x 32 query rows (256 rows per workgroup), two waves per SIMD:
//    Q stays in registers (64), and O is accumulated in two passes of 128
//    columns (64 registers), the scores being recomputed in the second
//    pass.  One pass holding all 256 columns needs ~400 registers, i.e. one
//    wave per SIMD and no partner to overlap the matrix and softmax phases.
//    Both passes run the same online softmax over the same scores, so their
//    running max and sum agree and each pass normalises its own columns.
//  * 32-key tiles.  A K tile is 32 rows of 512 bytes (16 KB); a pass's V
//    tile holds only that pass's 128 columns (32 rows of 256 bytes, 8 KB).
//  * K rows: 16-byte chunk q of row r is stored at chunk q ^ swz(r) (the
//    XOR touches the low four chunk bits, so chunks stay in their 256-byte
//    half).  The Sᵀ = K Qᵀ operand of step c (logical chunk 2c + lh of row
//    lr) then sits at base ^ 32c with one base per lane.  V rows use the
//    256-byte layout of the head_dim 128 core, so its Vᵀ transpose reads
//    carry over.
//  * DMA as in the head_dim 128 core: group A's four waves each fill 8
//    consecutive keys of K and of V through a buffer resource, from inside
//    their matrix phase.
#pragma once

#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

struct FwdShapeD256 {
  static constexpr int D = 256;
  static constexpr int DO = 128;              // O columns per pass
  static constexpr int NPASS = D / DO;
  static constexpr int BM = tiles::kFwd256Rows;   // query rows per workgroup
  static constexpr int BN = tiles::kFwd256Keys;   // keys per tile
  static constexpr int NW = tiles::kFwd256Waves;  // waves
  static constexpr int KROWB = 2 * D;          // bytes per K row
  static constexpr int VROWB = 2 * DO;         // bytes per V row of one pass
  static constexpr int KTILEB = BN * KROWB;    // 16 KB
  static constexpr int VTILEB = BN * VROWB;    // 8 KB
  static constexpr int LDS_BYTES = 2 * (KTILEB + VTILEB);
  static_assert(BN == 32 && NW == 8, "one 32-key block per tile, two wave groups of four");
};

// k0/v0 and k1/v1 are four distinct __shared__ arrays (KTILEB and VTILEB
// bytes); see attn_fwd_tile_d128 for the buffer rotation.
template <class T, class Prob>
__device__ __forceinline__ void attn_fwd_tile_d256(const Prob& P, int row0, float scale,
                                                   char* k0, char* v0, char* k1, char* v1) {
  using S = FwdShapeD256;
  constexpr int D = S::D, DO = S::DO, BN = S::BN;
  const float scale_log2 = scale * kLog2e;
  constexpr float kLazy = 8.f;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_id();
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
  // (2c + lh) ^ swz(lr) = 2c ^ (lh ^ swz(lr)), i.e. byte offset kbase ^ 32c.
  int kbase = lr * S::KROWB + 16 * (lh ^ swz_chunk(lr));
  // Vᵀ operand (as in attn_fwd_tile_d128, rows of VROWB bytes).
  int voff[2][DO / 32];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * hf;
    const int sw = swz_chunk(r);
#pragma unroll
    for (int dt = 0; dt < DO / 32; ++dt) {
      const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      voff[hf][dt] = r * S::VROWB + 16 * (chunk ^ sw) + 8 * (lane & 1);
    }
  }

  auto visible = [&](int n0) { return wave_active && n0 < w_hi_max && n0 + BN > w_lo_min; };
  f32x16 o[DO / 32];
  f32x16 s;
  u32x4 pb[BN / 16];
  float ms_run, l_run;
  int vcol = 0;  // first O / V column of the pass
  constexpr int kAheadS = FA_FWD_AHEAD_S, kAheadO = FA_FWD_AHEAD_O;

  auto gemm_s = [&](const char* kb) {
    asm volatile("" : "+v"(kbase));  // one base register, not one per step
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
    lds_pipeline<D / 16, kAheadS>(
        [&](int c) { return ld16(kb + (kbase ^ (32 * c))); },
        [&](int c, const u32x4& k) { s = T::mma32(k, qf[c], s); });
  };
  auto softmax = [&](int n0) {
    const bool need_mask = (n0 < w_lo_max) || (n0 + BN > w_hi_min);
    if (need_mask) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kv = n0 + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (kv < my_lo || kv >= my_hi) s[i] = neg_inf();
      }
    }
    float mt = neg_inf();
#pragma unroll
    for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[i]);
    mt = fmaxf(mt, swap_halves(mt)) * scale_log2;
    const bool grow = mt > ms_run + kLazy;
    if (__any(grow)) {
      const float ms_new = grow ? mt : ms_run;
      const float alpha = grow ? fast_exp2(ms_run - ms_new) : 1.f;
      ms_run = ms_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DO / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }
    const float mb = ms_run == neg_inf() ? 0.f : ms_run;
#pragma unroll
    for (int kc = 0; kc < BN / 16; ++kc)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e = 8 * kc + 2 * w;
        const float p0 = fast_exp2(fmaf(s[e], scale_log2, -mb));
        const float p1 = fast_exp2(fmaf(s[e + 1], scale_log2, -mb));
        pb[kc][w] = T::pack(p0, p1);
        l_run = T::sum2(p0, p1, pb[kc][w], l_run);
      }
  };
  auto gemm_o = [&](const char* vb) {
    struct VOps {
      u32x2 lo, hi;
    };
    lds_pipeline<(BN / 16) * (DO / 32), kAheadO>(
        [&](int k) {
          const int kc = k / (DO / 32), dt = k % (DO / 32);
          return VOps{lds_read_tr(vb + voff[0][dt] + kc * 16 * S::VROWB),
                      lds_read_tr(vb + voff[1][dt] + kc * 16 * S::VROWB)};
        },
        [&](int k, const VOps& r) {
          const int kc = k / (DO / 32), dt = k % (DO / 32);
          const u32x4 a = {r.lo[0], r.lo[1], r.hi[0], r.hi[1]};
          o[dt] = T::mma32(a, pb[kc], o[dt]);
        });
  };

  const bool grp_b = wave >= S::NW / 2;
  const int j0 = max(wg_lo, 0) / BN;
  const int j1 = (wg_hi + BN - 1) / BN;
  // DMA (group A, wave w < 4): keys n0 + 8w .. n0 + 8w + 7 of K (four 1 KB
  // blocks of 2 rows) and of the pass's V columns (two 1 KB blocks of 4
  // rows).  Lane offsets are relative to the wave's first row and fixed;
  // rows at or past wg_hi read as zero.
  constexpr int KB = 4, VB = 2;  // 1 KB blocks per DMA wave
  uint32_t k_loff[KB], v_loff[VB];
#pragma unroll
  for (int ii = 0; ii < KB; ++ii) {
    const int r8 = 2 * ii + (lane >> 5);
    const int r = 8 * wave + r8;  // row of the tile
    const uint32_t c = (lane & 31) ^ swz_chunk(r);
    k_loff[ii] = 2u * ((uint32_t)r8 * (uint32_t)P.k_row_stride() + 8u * c);
  }
#pragma unroll
  for (int ii = 0; ii < VB; ++ii) {
    const int r8 = 4 * ii + (lane >> 4);
    const int r = 8 * wave + r8;
    const uint32_t c = (lane & 15) ^ swz_chunk(r);
    v_loff[ii] = 2u * ((uint32_t)r8 * (uint32_t)P.v_row_stride() + 8u * c);
  }
  auto issue_rows = [&](int n0, char* dst, auto is_v) {
    constexpr bool kV = decltype(is_v)::value;
    const int nw = n0 + 8 * wave;
    const int nvalid = min(8, wg_hi - nw);  // n0 < wg_hi, so n0's row resolves
    const int nb = nvalid > 0 ? nw : n0;
    const uint16_t* base = kV ? P.v_ptr(nb) + vcol : P.k_ptr(nb);
    // K rows are read whole, V rows one pass's DO columns from vcol.
    const uint32_t bytes =
        span_bytes(nvalid, kV ? P.v_row_stride() : P.k_row_stride(), kV ? DO : D);
    u32x4 rs = rsrc_words(base, bytes);
#pragma unroll
    for (int w = 0; w < 4; ++w) rs[w] = __builtin_amdgcn_readfirstlane(rs[w]);
    if constexpr (kV) {
#pragma unroll
      for (int ii = 0; ii < VB; ++ii)
        buffer_lds16_opaque(rs, v_loff[ii], dst + (VB * wave + ii) * 1024);
    } else {
#pragma unroll
      for (int ii = 0; ii < KB; ++ii)
        buffer_lds16_opaque(rs, k_loff[ii], dst + (KB * wave + ii) * 1024);
    }
  };
  auto issue_k = [&](int n0, char* kb) { issue_rows(n0, kb, BoolC<false>{}); };
  auto issue_v = [&](int n0, char* vb) { issue_rows(n0, vb, BoolC<true>{}); };
  auto mma_phase = [&](int j, const char* vprev, const char* kcur, char* knext, char* vcur,
                       auto dma) {
    constexpr bool kDma = decltype(dma)::value;
    if (j - 1 >= j0 && visible((j - 1) * BN)) gemm_o(vprev);
    if (kDma && j + 1 < j1) issue_k((j + 1) * BN, knext);
    if (j < j1 && visible(j * BN)) gemm_s(kcur);
    if (kDma && j < j1) issue_v(j * BN, vcur);
  };
  auto sm_phase = [&](int js) {
    if (js >= j0 && js < j1 && visible(js * BN)) softmax(js * BN);
  };
  auto tile_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  auto run = [&](auto group_b) {
    constexpr bool kB = decltype(group_b)::value;
    constexpr BoolC<!kB> dma{};
    for (int j = j0;; j += 2) {
      if (kB) sm_phase(j - 1); else mma_phase(j, v1, k0, k1, v0, dma);
      if (kB) mma_phase(j, v1, k0, k1, v0, dma); else sm_phase(j);
      tile_barrier();
      if (j + 1 > j1) break;
      if (kB) sm_phase(j); else mma_phase(j + 1, v0, k1, k0, v1, dma);
      if (kB) mma_phase(j + 1, v0, k1, k0, v1, dma); else sm_phase(j + 1);
      tile_barrier();
      if (j + 2 > j1) break;
    }
  };

  // Every wave runs both passes (their barriers pair up); the last barrier
  // of a pass also frees the buffers for the next pass's first DMA.
#pragma unroll 1
  for (int pass = 0; pass < S::NPASS; ++pass) {
    vcol = pass * DO;
#pragma unroll
    for (int dt = 0; dt < DO / 32; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
    ms_run = neg_inf();
    l_run = 0.f;
    if (j0 < j1 && !grp_b) issue_k(j0 * BN, k0);
    wait_vmem();
    __syncthreads();
    if (grp_b)
      run(BoolC<true>{});
    else
      run(BoolC<false>{});
    const float l_all = l_run + swap_halves(l_run);
    if (row_valid) fwd_store_row<T>(P, row, lh, o, l_all, ms_run, vcol);
  }
}

}  // namespace fa
