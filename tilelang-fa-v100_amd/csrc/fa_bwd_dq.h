// dQ of the dense attention backward (head_dim 64 / 128 / 256).
//
// Replaces the reference's query-stationary dQ kernel
// (tilelang_fa_v100/_kernels_backward.py:10-85): every dQ row is built by one
// wave over all keys its query sees and written once, so the result does not
// depend on the order in which workgroups run (no atomics).  The key-
// stationary kernels (bwd_main_kernel, bwd_main_mfma_kernel) compute dK / dV.
//
// Per 32-query-row wave and BN-key tile, with the same register layout as
// the forward's Oᵀ = Vᵀ Pᵀ (fa_fwd_d128.h), so that no score leaves the
// registers:
//   Sᵀ  = K Qᵀ      (A = K rows from LDS, B = the wave's Q rows in registers)
//   dPᵀ = V dOᵀ     (A = V rows from LDS, B = the wave's dO rows)
//   P = exp2(Sᵀ·scale·log2e − LSE·log2e),  dSᵀ = P (dPᵀ − rowdot)·scale
//   (rounded to 16 bits with the scale in, as the reference does,
//   _kernels_backward.py:74)
//   dQᵀ += Kᵀ dSᵀ   (A = Kᵀ by ds_read_b64_tr_b16 from the same K tile,
//                    B = dSᵀ packed straight from the accumulators)
// A lane's scores all belong to its own query row (column lr of Sᵀ), so the
// row statistics (LSE·log2e, scale·rowdot, computed here) are one register
// each.  K and V tiles go HBM -> LDS with global_load_lds_dwordx4 (every
// wave loads BPW 1 KB blocks of each, two tiles in flight), rows stored
// with the 16-byte chunk swizzle of fa_fwd_d128.h.
#pragma once

#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

template <int D_>
struct BwdDqShape {
  static constexpr int D = D_;
  static constexpr int NW = D == 256 ? 4 : 8;  // waves (one per SIMD at D = 256)
  static constexpr int BM = 32 * NW;           // query rows per workgroup
  static constexpr int BN = D == 256 ? 32 : 64;  // keys per tile
  static constexpr int ROWB = 2 * D;           // bytes per K / V row
  static constexpr int CPR = D / 8;            // 16-byte chunks per row
  static constexpr int RPB = 1024 / ROWB;      // rows per 1 KB DMA block
  static constexpr int TILEB = BN * ROWB;      // 8 KB (D = 64) or 16 KB per K or V tile
  static constexpr int BPW = TILEB / 1024 / NW;  // DMA blocks per wave and tile
  static constexpr int WPE = NW / 4;           // waves per SIMD
  // Chunk swizzle bits: all four for rows of 16 or more chunks (the low four
  // bits of each 256-byte half at D = 256), three for 8-chunk rows.
  static constexpr int SWZ_MASK = CPR >= 16 ? 15 : CPR - 1;
  static_assert(BPW * NW * 1024 == TILEB, "DMA split");
};

template <class T, int D_, int MODE>
__global__ __launch_bounds__((64 * BwdDqShape<D_>::NW), (BwdDqShape<D_>::WPE))
void bwd_dq_kernel(fa_bwd_args a, float* stats) {
  using S = BwdDqShape<D_>;
  constexpr int D = S::D, BN = S::BN;
  __shared__ __attribute__((aligned(16))) char k0[S::TILEB], v0[S::TILEB], k1[S::TILEB],
      v1[S::TILEB];

  const int Sq = a.seqlen_q, Sk = a.seqlen_k, H = a.num_heads;
  const int qtiles = (Sq + S::BM - 1) / S::BM;
  const TileHead th = xcd_tile_order(blockIdx.x, qtiles, a.batch * H);
  const int bh = th.bh;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.num_heads_k);
  // Heaviest causal tiles (largest query index) first.
  const int qt = MODE != kMaskNone ? qtiles - 1 - th.rank : th.rank;
  const int row0 = qt * S::BM;
  const Band band = mode_band<MODE>(a);
  // Row r sees keys [kv_lo(r), kv_hi(r)) (band clipped to [0, Sk)).
  auto kv_lo = [&](int r) { return band.wl >= 0 ? min(max(r + band.off - band.wl, 0), Sk) : 0; };
  auto kv_hi = [&](int r) {
    return band.wr >= 0 ? min(max(r + band.off + band.wr + 1, 0), Sk) : Sk;
  };

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  const float scale_log2 = a.softmax_scale * kLog2e;
  const float sc = a.softmax_scale;

  const int row_last = min(row0 + S::BM, Sq) - 1;
  const int wg_lo = kv_lo(row0), wg_hi = kv_hi(row_last);
  const int wrow0 = row0 + 32 * wave;
  const bool wave_active = wrow0 < Sq;
  const int wrow_last = min(wrow0 + 31, Sq - 1);
  const int w_lo_min = wave_active ? kv_lo(wrow0) : 0;
  const int w_lo_max = wave_active ? kv_lo(wrow_last) : 0;
  const int w_hi_min = wave_active ? kv_hi(wrow0) : 0;
  const int w_hi_max = wave_active ? kv_hi(wrow_last) : 0;
  const int row = wrow0 + lr;
  const bool row_valid = row < Sq;
  const int my_lo = row_valid ? kv_lo(row) : 0;
  const int my_hi = row_valid ? kv_hi(row) : 0;

  // ---- this lane's query row: Q and dO as B operands, and its statistics,
  // computed here and stored for the dK / dV kernel, which runs after this
  // one: LSE·log2(e) (+inf for a row that saw no key, and for rows past Sq,
  // so that P is exactly zero) and scale·rowdot, rowdot = Σ_d O·dO (the
  // reference's row_dot, _kernels_backward.py:203).  Lanes l and l + 32 hold the two
  // halves of each 16-column chunk of the row.
  u32x4 qf[D / 16], df[D / 16];
  float lse2 = __builtin_inff(), rdot = 0.f;
  {
    const int64_t r = min(row, Sq - 1);
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.q_stride[0] +
                         h * a.q_stride[2] + r * a.q_stride[1];
    const uint16_t* dp = static_cast<const uint16_t*>(a.dout) + b * a.do_stride[0] +
                         h * a.do_stride[2] + r * a.do_stride[1];
    const uint16_t* op = static_cast<const uint16_t*>(a.out) + b * a.o_stride[0] +
                         h * a.o_stride[2] + r * a.o_stride[1];
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      qf[c] = ld16(qp + 16 * c + 8 * lh);
      df[c] = ld16(dp + 16 * c + 8 * lh);
      const u32x4 ov = ld16(op + 16 * c + 8 * lh);
#pragma unroll
      for (int w = 0; w < 4; ++w) part = T::dot2(ov[w], df[c][w], part);
    }
    const float full = half_sum(part);
    if (row_valid) {
      const float l = a.lse[(int64_t)bh * Sq + row];
      lse2 = (l == neg_inf()) ? __builtin_inff() : l * kLog2e;
      rdot = full * sc;
      if (lh == 0) {
        float* st = stats + 2 * (int64_t)bh * Sq;
        st[row] = lse2;
        st[Sq + row] = rdot;
      }
    }
  }

  // ---- per-lane LDS offsets.  Row read (A of Sᵀ and dPᵀ), chunk c: row lr
  // (+32 kt), logical chunk 2c + lh.  Transpose read (A of dQᵀ), 16-key
  // chunk kc, d tile dt: rows 16kc + 4(lane/32) + (lane%16)/4 (+8 for the
  // upper half), columns 32dt + 16((lane/16)%2) + 4(lane%4).  The swizzle of
  // a row depends on the row modulo 16 only, so kc and kt are immediates.
  auto swz = [](int r) { return swz_chunk(r) & S::SWZ_MASK; };
  int koff[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) koff[c] = lr * S::ROWB + 16 * ((2 * c + lh) ^ swz(lr));
  int toff[2][D / 32];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * hf;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      toff[hf][dt] = r * S::ROWB + 16 * (chunk ^ swz(r)) + 8 * (lane & 1);
    }
  }

  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;
  // D = 256: the dQ accumulators (32 rows x 256 d, 128 registers) stay in
  // AGPRs (mma32_agpr) and Q / dO rows, scores and operands in VGPRs.
  if constexpr (D == 256) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) agpr_fence_in(acc[dt]);
  }

  // ---- tile loader: wave w fills 1 KB blocks BPW w .. BPW w + BPW - 1 of
  // the K and V tiles, i.e. the tile's rows WR w .. WR w + WR - 1; lane l of
  // block blk holds row RPB blk + l / CPR, stored chunk l % CPR (logical
  // chunk (l % CPR) ^ swz(row)).  The rows go through buffer resources based
  // at the wave's first row: the lane's byte offset is fixed for the whole
  // loop (below 8 rows, so 32 bits hold it for any sequence stride below
  // 2^26), and rows at or past the last key read as zero (their scores are
  // masked).
  constexpr int WR = S::RPB * S::BPW;
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[2];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[2];
  uint32_t k_loff[S::BPW], v_loff[S::BPW];
#pragma unroll
  for (int ii = 0; ii < S::BPW; ++ii) {
    const int rr = S::RPB * ii + lane / S::CPR;  // row within the wave's WR rows
    const int c = (lane % S::CPR) ^ swz(WR * wave + rr);
    k_loff[ii] = 2u * (rr * (uint32_t)a.k_stride[1] + 8 * c);
    v_loff[ii] = 2u * (rr * (uint32_t)a.v_stride[1] + 8 * c);
  }
  const int j0 = max(wg_lo, 0) / BN;
  const int j1 = (wg_hi + BN - 1) / BN;
  // Tiles are issued in order (n0 = j0 BN, (j0 + 1) BN, ...), so the two
  // resources are carried from tile to tile: one 64-bit add of the base
  // words each, num_records recomputed only where the rows run past wg_hi.
  const uint32_t k_full = span_bytes(WR, a.k_stride[1], D), v_full = span_bytes(WR, a.v_stride[1], D);
  const int nb0 = j0 * BN + WR * wave;
  u32x4 rk = rsrc_words(kg + (int64_t)nb0 * a.k_stride[1], k_full);
  u32x4 rv = rsrc_words(vg + (int64_t)nb0 * a.v_stride[1], v_full);
  auto step_rsrc = [](u32x4& r, uint64_t bytes) {
    const uint64_t p = (((uint64_t)r[1]) << 32 | r[0]) + bytes;
    r[0] = (uint32_t)p;
    r[1] = (uint32_t)(p >> 32);
  };
  auto issue_tile = [&](int n0, char* kb, char* vb) {
    const int nb = n0 + WR * wave;
    u32x4 k = rk, v = rv;
    if (nb + WR > wg_hi) {
      const uint32_t nvalid = (uint32_t)max(min(WR, wg_hi - nb), 0);
      k[2] = span_bytes(nvalid, a.k_stride[1], D);
      v[2] = span_bytes(nvalid, a.v_stride[1], D);
    }
#pragma unroll
    for (int ii = 0; ii < S::BPW; ++ii) {
      const int blk = S::BPW * wave + ii;
      buffer_lds16_opaque(k, k_loff[ii], kb + blk * 1024);
      buffer_lds16_opaque(v, v_loff[ii], vb + blk * 1024);
    }
    step_rsrc(rk, 2ull * BN * (uint64_t)a.k_stride[1]);
    step_rsrc(rv, 2ull * BN * (uint64_t)a.v_stride[1]);
  };

  // One tile, as BN / 32 blocks of 32 keys: each block's scores, P / dS and
  // dQ products before the next block's (halves the live accumulators).
  auto compute_tile = [&](int n0, const char* kb, const char* vb) {
    if (!(wave_active && n0 < w_hi_max && n0 + BN > w_lo_min)) return;
    const bool need_mask = (n0 < w_lo_max) || (n0 + BN > w_hi_min);
#pragma unroll
    for (int kt = 0; kt < BN / 32; ++kt) {
      // Sᵀ first; then each dPᵀ product is followed by 16 / (D / 16)
      // elements of P, so the exponentials issue while the matrix core works
      // through dPᵀ (the two chains interleaved left them to run after both).
      const int ko = kt * 32 * S::ROWB;
      f32x16 s, dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) s = T::mma32(ld16(kb + koff[c] + ko), qf[c], s);
      sched_pipeline<D / 16, 1, 1, 2>();
      // P and dS; element i is key n0 + 32kt + 8(i/4) + 4lh + i%4.
      auto probs = [&](auto masked) {
        constexpr bool kMasked = decltype(masked)::value;
#pragma unroll
        for (int i = 0; i < 16; ++i) dp[i] = 0.f;
        auto prob = [&](int i) {
          float p = fast_exp2(fmaf(s[i], scale_log2, -lse2));
          if constexpr (kMasked) {
            const int kv = n0 + kt * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
            p = (kv >= my_lo && kv < my_hi) ? p : 0.f;
          }
          s[i] = p;
        };
        constexpr int EPC = 16 / (D / 16) > 0 ? 16 / (D / 16) : 1;
        lds_pipeline<D / 16, 2>([&](int c) { return ld16(vb + koff[c] + ko); },
                                [&](int c, const u32x4& av) {
                                  dp = T::mma32(av, df[c], dp);
#pragma unroll
                                  for (int e = 0; e < EPC; ++e)
                                    if (EPC * c + e < 16) prob(EPC * c + e);
                                });
#pragma unroll
        for (int i = EPC * (D / 16); i < 16; ++i) prob(i);
#pragma unroll
        for (int i = 0; i < 16; ++i) dp[i] = s[i] * fmaf(dp[i], sc, -rdot);
      };
      if (need_mask)
        probs(BoolC<true>{});
      else
        probs(BoolC<false>{});
      // dSᵀ as the B operand of dQᵀ += Kᵀ dSᵀ, 16-key chunks kc = 2kt, 2kt+1.
      u32x4 sb[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int e = 8 * h2 + 2 * w;
          sb[h2][w] = T::pack(dp[e], dp[e + 1]);
        }
      struct KtOps {
        u32x2 lo, hi;
      };
      lds_pipeline<2 * (D / 32), 2>(
          [&](int k) {
            const int kc = 2 * kt + k / (D / 32), dt = k % (D / 32);
            return KtOps{lds_read_tr(kb + toff[0][dt] + kc * 16 * S::ROWB),
                         lds_read_tr(kb + toff[1][dt] + kc * 16 * S::ROWB)};
          },
          [&](int k, const KtOps& r) {
            const int dt = k % (D / 32);
            const u32x4 ak = {r.lo[0], r.lo[1], r.hi[0], r.hi[1]};
            if constexpr (D == 256)
              mma32_agpr<T>(acc[dt], ak, sb[k / (D / 32)]);
            else
              acc[dt] = T::mma32(ak, sb[k / (D / 32)], acc[dt]);
          });
    }
  };

  // Double-buffered tiles; the loop covers two tiles so that every LDS read
  // names one array pair while the DMA of the next tile targets the other.
  if (j0 < j1) issue_tile(j0 * BN, k0, v0);
  for (int j = j0; j < j1; j += 2) {
    wait_vmem();
    __syncthreads();  // tile j resident; every wave is done with tile j - 1
    if (j + 1 < j1) issue_tile((j + 1) * BN, k1, v1);
    compute_tile(j * BN, k0, v0);
    if (j + 1 >= j1) break;
    wait_vmem();
    __syncthreads();
    if (j + 2 < j1) issue_tile((j + 2) * BN, k0, v0);
    compute_tile((j + 1) * BN, k1, v1);
  }

  // ---- dQ = Σ dS K; acc[dt][4g + r] = dQ[row][32dt + 8g + 4lh + r].
  if constexpr (D == 256) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) agpr_fence_out(acc[dt]);
  }
  if (!row_valid) return;
  uint16_t* dqp = static_cast<uint16_t*>(a.dq) + b * a.dq_stride[0] +
                  (int64_t)row * a.dq_stride[1] + h * a.dq_stride[2];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w[0] = T::pack(acc[dt][4 * g], acc[dt][4 * g + 1]);
      w[1] = T::pack(acc[dt][4 * g + 2], acc[dt][4 * g + 3]);
      st8(dqp + 32 * dt + 8 * g + 4 * lh, w);
    }
}

}  // namespace fa
