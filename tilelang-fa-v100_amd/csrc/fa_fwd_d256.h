// Attention forward core for head_dim 256 on gfx950 (dense rows, and paged
// rows with pages of at least 16 keys): 4 waves x 32 query rows (128 rows
// per workgroup), one wave per SIMD, 32-key tiles.
//  * O (32 rows x 256 d, 128 registers) lives in AGPRs for the whole tile
//    (mma32_agpr), Q (64) and the scores in VGPRs: one pass over the keys
//    with 512 registers per wave.  (Two waves per SIMD would need O in two
//    128-column passes with the scores recomputed, 1.5x the products.)
//  * Software pipeline inside the wave: the scores of tile j + 1 are
//    computed while tile j is exponentiated (the max, rescale decision and
//    exponentials are spread between the 16 products of Sᵀ(j + 1)), then
//    Oᵀ += Vᵀ(j) Pᵀ(j).  The wave's matrix core has no partner wave to
//    overlap with, so the overlap has to come from its own instruction
//    stream.
//  * K and V tiles are 32 rows of 512 bytes; 16-byte chunk q of row r is
//    stored at chunk q ^ swz(r), the XOR touching the low four chunk bits
//    (chunks stay in their 256-byte half).  Double buffered: iteration j
//    reads K(j + 1) and V(j) while K(j + 2) and V(j + 1) stream in.  Each
//    wave DMAs 8 rows of each (four 1 KB blocks) through a buffer resource.
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

// k0/v0/k1/v1: four distinct __shared__ arrays of TILEB bytes.
template <class T, class Prob>
__device__ __forceinline__ void attn_fwd_tile_d256(const Prob& P, int row0, float scale,
                                                   char* k0, char* v0, char* k1, char* v1) {
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
  auto gemm_o = [&](const char* vb) {
    asm volatile("" : "+v"(vbase[0]), "+v"(vbase[1]));
    struct VOps {
      u32x2 lo, hi;
    };
    lds_pipeline<(BN / 16) * (D / 32), kAheadO>(
        [&](int k) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          const int ro = kc * 16 * S::ROWB;
          return VOps{lds_read_tr(vb + (vbase[0] ^ (64 * dt)) + ro),
                      lds_read_tr(vb + (vbase[1] ^ (64 * dt)) + ro)};
        },
        [&](int k, const VOps& r) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          mma32_agpr<T>(o[dt], u32x4{r.lo[0], r.lo[1], r.hi[0], r.hi[1]}, pb[kc]);
        });
  };

  // DMA: wave w fills rows 8w .. 8w + 7 of a K or V tile (blocks 4w .. 4w+3,
  // two rows per 1 KB block); lane offsets are fixed, rows at or past wg_hi
  // read as zero.
  uint32_t k_loff[4], v_loff[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int r8 = 2 * ii + (lane >> 5);
    const uint32_t c = (lane & 31) ^ swz_chunk(8 * wave + r8);
    k_loff[ii] = 2u * ((uint32_t)r8 * (uint32_t)P.k_row_stride() + 8u * c);
    v_loff[ii] = 2u * ((uint32_t)r8 * (uint32_t)P.v_row_stride() + 8u * c);
  }
  auto issue_rows = [&](int n0, char* dst, auto is_v) {
    constexpr bool kV = decltype(is_v)::value;
    const int nw = n0 + 8 * wave;
    const int nvalid = min(8, wg_hi - nw);  // n0 < wg_hi, so n0's row resolves
    const int nb = nvalid > 0 ? nw : n0;
    const uint16_t* base = kV ? P.v_ptr(nb) : P.k_ptr(nb);
    const uint32_t bytes = span_bytes(nvalid, kV ? P.v_row_stride() : P.k_row_stride(), D);
    u32x4 rs = rsrc_words(base, bytes);
#pragma unroll
    for (int w = 0; w < 4; ++w) rs[w] = __builtin_amdgcn_readfirstlane(rs[w]);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      buffer_lds16_opaque(rs, kV ? v_loff[ii] : k_loff[ii], dst + (4 * wave + ii) * 1024);
  };
  auto tile_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Iteration j: K(j + 1) in kn, V(j) in vc; DMA of K(j + 2) into kd and of
  // V(j + 1) into vd; cur holds Sᵀ(j), nxt receives Sᵀ(j + 1).
  const int j0 = max(wg_lo, 0) / BN;
  const int j1 = (wg_hi + BN - 1) / BN;
  auto step = [&](int j, const char* kn, const char* vc, char* kd, char* vd, f32x16& cur,
                  f32x16& nxt) {
    tile_barrier();
    if (j + 2 < j1) issue_rows((j + 2) * BN, kd, BoolC<false>{});
    if (j + 1 < j1) issue_rows((j + 1) * BN, vd, BoolC<true>{});
    const bool vis = visible(j);
    const bool vis_n = j + 1 < j1 && visible(j + 1);
    if (!vis) {
      if (vis_n) gemm_s(nxt, kn, [](int) {});
      return;
    }
    const int n0 = j * BN;
    if ((n0 < w_lo_max) || (n0 + BN > w_hi_min)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kv = n0 + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (kv < my_lo || kv >= my_hi) cur[i] = neg_inf();
      }
    }
    // The online-softmax update of tile j in 14 slices: row max (steps
    // 0-3), the other half-row's max (4), rescale decision (5), then one
    // pair of probabilities per step (6-13).
    float mt = neg_inf(), alpha = 1.f, mb = 0.f;
    bool grow = false;
    auto slice = [&](int c) {
      if (c < 4) {
#pragma unroll
        for (int i = 4 * c; i < 4 * c + 4; ++i) mt = fmaxf(mt, cur[i]);
      } else if (c == 4) {
        mt = half_max(mt) * scale_log2;
      } else if (c == 5) {
        // A row's max only moves when the tile max exceeds it by more than
        // kLazy, so P <= 2^kLazy and O is rescaled on few tiles.
        grow = mt > ms_run + kLazy;
        const float ms_new = grow ? mt : ms_run;
        alpha = grow ? fast_exp2(ms_run - ms_new) : 1.f;
        ms_run = ms_new;
        l_run *= alpha;
        // A row with no visible key so far has ms_run = -inf and only -inf
        // scores in this tile: any finite offset gives P = 0.
        mb = ms_run == neg_inf() ? 0.f : ms_run;
      } else if (c < 14) {
        const int pr = c - 6, e = 2 * pr;
        const float p0 = fast_exp2(fmaf(cur[e], scale_log2, -mb));
        const float p1 = fast_exp2(fmaf(cur[e + 1], scale_log2, -mb));
        pb[pr >> 2][pr & 3] = T::pack(p0, p1);
        l_run = T::sum2(p0, p1, pb[pr >> 2][pr & 3], l_run);
      }
    };
    if (vis_n) {
      gemm_s(nxt, kn, slice);
    } else {
#pragma unroll
      for (int c = 0; c < 14; ++c) slice(c);
    }
    if (o_live && __any(grow)) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        agpr_fence_out(o[dt]);
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
      }
    }
    gemm_o(vc);
    o_live = true;
  };

  if (j0 < j1) {
    f32x16 sa, sb;
    issue_rows(j0 * BN, k0, BoolC<false>{});
    tile_barrier();
    if (j0 + 1 < j1) issue_rows((j0 + 1) * BN, k1, BoolC<false>{});
    issue_rows(j0 * BN, v0, BoolC<true>{});
    if (visible(j0)) gemm_s(sa, k0, [](int) {});
    for (int j = j0;; j += 2) {
      step(j, k1, v0, k0, v1, sa, sb);
      if (j + 1 >= j1) break;
      step(j + 1, k0, v1, k1, v0, sb, sa);
      if (j + 2 >= j1) break;
    }
  }

#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) agpr_fence_out(o[dt]);
  const float l_all = half_sum(l_run);
  if (row_valid) fwd_store_row<T>(P, row, lh, o, l_all, ms_run);
}

}  // namespace fa
