// Online-softmax attention forward for one 128-row query tile (gfx950).
//
// Algorithm (FlashAttention-2 forward, as in the reference
// tilelang_fa_v100/_kernels_forward.py:94-172 and the paged variant
// _kernels_paged.py:193-344): for each key tile, S = Q K^T (fp32 MFMA
// accumulate), running row max m and row sum l, O <- O * exp(m_old - m_new)
// + exp(S - m_new) V, and in the epilogue O / l and LSE = m * scale + ln l.
//
// Layout choices (see fa_common.h for the MFMA lane layout):
//  * Four waves per workgroup; wave w owns query rows row0 + 32w .. +31 and
//    lane (lr, lh) owns query row row0 + 32w + lr.
//  * The kernel computes S^T = K Q^T (A = K from LDS, B = Q in registers), so
//    every score a lane holds belongs to its own query row.  The row max
//    therefore needs a single exchange with lane ^ 32 and the row sum none.
//  * The probabilities P^T are kept in registers and used directly as the B
//    operand of O^T = V^T P^T; V is stored transposed in LDS (keys
//    contiguous) so the A operand is two 8-byte LDS reads.
//  * K and V^T tiles are double-buffered in LDS; the next tile's global loads
//    are issued before the current tile's MFMAs (one barrier per tile).
//  * Visibility of key n to row r is an interval [kv_lo(r), kv_hi(r)) that is
//    non-decreasing in r.  That covers dense causal (bottom-right), the paged
//    prefix-anchored causal mask, sliding windows and plain length limits,
//    and lets whole tiles be skipped or left unmasked from two row bounds.
#pragma once

#include "fa_common.h"

namespace fa {

template <int D>
struct FwdShape {
  static constexpr int BM = tiles::kFwdCoreRows;  // query rows per workgroup
  // keys per tile (64 for D=128)
  static constexpr int BN = D <= 256 ? tiles::kFwdCoreTileElems / D : tiles::kFwdCoreKeys512;
  static constexpr int KS = D + 8;         // LDS row stride of K, elements
  static constexpr int VS = BN + 4;        // LDS row stride of V^T, elements
  static constexpr int KT = BN / 32;       // 32-key sub-tiles of S^T
  static constexpr int DC = D / 16;        // 16-wide d chunks (QK^T)
  // O columns per pass: D up to 256; D = 512 runs two passes over the keys,
  // each accumulating 256 columns of O (the scores are recomputed), so that
  // Q, O and the tile staging fit one wave's 512 registers.
  static constexpr int DO = D <= 256 ? D : 256;
  static constexpr int NPASS = D / DO;
  static constexpr int DT = DO / 32;       // 32-wide d tiles of O^T per pass
  static constexpr int KC = BN / 16;       // 16-key chunks (PV)
  static constexpr int CPR = D / 8;        // 16-byte chunks per K row
  static constexpr int RSTEP = 256 / CPR;  // rows between a thread's K chunks
  static constexpr int NK = BN * CPR / 256;  // 16-byte K chunks per thread per tile
  static constexpr int CPRV = DO / 8;      // 16-byte chunks per V row and pass
  static constexpr int RSTEPV = 256 / CPRV;
  static constexpr int NV = BN * CPRV / 256;  // 16-byte V chunks per thread per tile
  static constexpr int VG = 4 * RSTEPV;    // keys between a thread's groups of 4 V rows
  static constexpr int LDS_ELEMS = 2 * BN * KS + 2 * DO * VS;
  // Two workgroups per CU (2 waves per SIMD) fit the register file up to D=128.
  static constexpr int kWavesPerEU = D <= 128 ? 2 : 1;
  static_assert(BN % 32 == 0 && D % 32 == 0, "tile shape");
  static_assert(NV % 4 == 0 && BN % VG == 0 && NK * 256 == BN * CPR,
                "whole groups of four V rows per thread");
};

// Prob must provide:
//   int nrows;
//   int kv_lo(int r), kv_hi(int r)      visible keys of valid row r
//   const uint16_t* q_ptr(int r); uint16_t* o_ptr(int r); float* lse_ptr(int r)
//   bool has_lse;
//   const uint16_t* k_ptr(int n); const uint16_t* v_ptr(int n)
template <class T, int D, class Prob>
__device__ __forceinline__ void attn_fwd_tile(const Prob& P, int row0,
                                              float scale, uint16_t* smem) {
  using S = FwdShape<D>;
  const float scale_log2 = scale * kLog2e;
  constexpr float kLazy = 8.f;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;

  uint16_t* Ks = smem;                    // [2][BN][KS]
  uint16_t* Vt = smem + 2 * S::BN * S::KS;  // [2][DO][VS]

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

  // Q rows straight from HBM into the B-operand layout.
  u32x4 qf[S::DC];
  {
    const uint16_t* qp = row_valid ? P.q_ptr(row) : nullptr;
#pragma unroll
    for (int c = 0; c < S::DC; ++c)
      qf[c] = row_valid ? ld16(qp + 16 * c + 8 * lh) : u32x4{0, 0, 0, 0};
  }

  f32x16 o[S::DT];
  float ms_run, l_run;  // running row max * scale * log2(e), running row sum

  // Cooperative tile loader: thread t owns the 16-byte column chunk
  // col8 = t % CPR; K rows r0 + i*RSTEP and V rows 4*r0 + i (four consecutive
  // keys, so V can be transposed in registers before the LDS store).
  const int col8 = tid % S::CPR;
  const int r0 = tid / S::CPR;
  const int col8v = tid % S::CPRV;
  const int r0v = tid / S::CPRV;
  u32x4 kreg[S::NK], vreg[S::NV];
  int vcol = 0;  // first O / V column of the pass
  // Rows at or beyond wg_hi are never visible: they are loaded from the last
  // visible row instead (finite data, multiplied by P = 0), which keeps every
  // load unconditional and never touches memory past the keys.
  const int ld_last = max(wg_hi - 1, 0);

  auto load_tile = [&](int n0) {
#pragma unroll
    for (int i = 0; i < S::NK; ++i) {
      const int n = min(n0 + r0 + i * S::RSTEP, ld_last);
      kreg[i] = ld16(P.k_ptr(n) + col8 * 8);
    }
#pragma unroll
    for (int i = 0; i < S::NV; ++i) {
      const int n = min(n0 + (i / 4) * S::VG + 4 * r0v + (i % 4), ld_last);
      vreg[i] = ld16(P.v_ptr(n) + vcol + col8v * 8);
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* kb = Ks + buf * S::BN * S::KS;
#pragma unroll
    for (int i = 0; i < S::NK; ++i)
      st16(kb + (r0 + i * S::RSTEP) * S::KS + col8 * 8, kreg[i]);
    uint16_t* vb = Vt + buf * S::DO * S::VS;
#pragma unroll
    for (int gi = 0; gi < S::NV / 4; ++gi)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int w = j >> 1;
        const u32x4* vg = vreg + 4 * gi;
        u32x2 pr;
        if (j & 1) {
          pr[0] = pack_hi(vg[0][w], vg[1][w]);
          pr[1] = pack_hi(vg[2][w], vg[3][w]);
        } else {
          pr[0] = pack_lo(vg[0][w], vg[1][w]);
          pr[1] = pack_lo(vg[2][w], vg[3][w]);
        }
        st8(vb + (col8v * 8 + j) * S::VS + gi * S::VG + 4 * r0v, pr);
      }
  };

  const int j0 = max(wg_lo, 0) / S::BN;
  const int j1 = (wg_hi + S::BN - 1) / S::BN;
  for (int pass = 0; pass < S::NPASS; ++pass) {
  vcol = pass * S::DO;
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  ms_run = neg_inf();
  l_run = 0.f;
  if (j0 < j1) {
    load_tile(j0 * S::BN);
    store_tile(0);
    __syncthreads();
    for (int j = j0; j < j1; ++j) {
      const int buf = (j - j0) & 1;
      const bool more = j + 1 < j1;
      if (more) load_tile((j + 1) * S::BN);
      const int n0 = j * S::BN;
      if (wave_active && n0 < w_hi_max && n0 + S::BN > w_lo_min) {
        const uint16_t* kb = Ks + buf * S::BN * S::KS;
        const uint16_t* vb = Vt + buf * S::DO * S::VS;
        f32x16 s[S::KT];
#pragma unroll
        for (int kt = 0; kt < S::KT; ++kt) {
#pragma unroll
          for (int i = 0; i < 16; ++i) s[kt][i] = 0.f;
#pragma unroll
          for (int c = 0; c < S::DC; ++c) {
            const u32x4 a = ld16(kb + (kt * 32 + lr) * S::KS + 16 * c + 8 * lh);
            s[kt] = T::mma32(a, qf[c], s[kt]);
          }
        }
        const bool need_mask = (n0 < w_lo_max) || (n0 + S::BN > w_hi_min);
        if (need_mask) {
#pragma unroll
          for (int kt = 0; kt < S::KT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int kv = n0 + kt * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
              if (kv < my_lo || kv >= my_hi) s[kt][i] = neg_inf();
            }
        }
        // Running max in scaled base-2 units (ms).  A row's max only moves
        // when the tile max exceeds it by more than kLazy, so P <= 2^kLazy
        // (exact in fp16/bf16) and O is rescaled on few tiles.
        float mt = neg_inf();
#pragma unroll
        for (int kt = 0; kt < S::KT; ++kt)
#pragma unroll
          for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[kt][i]);
        mt = half_max(mt) * scale_log2;
        const bool grow = mt > ms_run + kLazy;
        if (__any(grow)) {
          const float ms_new = grow ? mt : ms_run;
          const float alpha = grow ? fast_exp2(ms_run - ms_new) : 1.f;
          ms_run = ms_new;
          l_run *= alpha;
#pragma unroll
          for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
        }
        // A row with no visible key so far has ms_run = -inf and only -inf
        // scores in this tile: any finite offset gives P = 0.
        const float mb = ms_run == neg_inf() ? 0.f : ms_run;
        // P^T chunk kc holds keys 16kc + 8*(j/4) + 4*lh + (j%4), j = 0..7,
        // which are accumulator entries 8*(kc%2) + j of sub-tile kc/2.
        u32x4 pb[S::KC];
#pragma unroll
        for (int kc = 0; kc < S::KC; ++kc)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int e = 8 * (kc & 1) + 2 * w;
            const float p0 = fast_exp2(fmaf(s[kc >> 1][e], scale_log2, -mb));
            const float p1 = fast_exp2(fmaf(s[kc >> 1][e + 1], scale_log2, -mb));
            pb[kc][w] = T::pack(p0, p1);
            l_run = T::sum2(p0, p1, pb[kc][w], l_run);
          }
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
          for (int kc = 0; kc < S::KC; ++kc) {
            const uint16_t* vr = vb + (dt * 32 + lr) * S::VS + 16 * kc + 4 * lh;
            const u32x2 lo8 = ld8(vr);
            const u32x2 hi8 = ld8(vr + 8);
            const u32x4 a = {lo8[0], lo8[1], hi8[0], hi8[1]};
            o[dt] = T::mma32(a, pb[kc], o[dt]);
          }
      }
      if (more) store_tile(buf ^ 1);
      __syncthreads();
    }
  }

  // Epilogue: both halves of the wave hold partial sums of the same row.
  // (No early return: a second pass still takes part in the barriers.)
  const float l_all = half_sum(l_run);
  if (row_valid) fwd_store_row<T>(P, row, lh, o, l_all, ms_run, vcol);
  }  // pass
}

}  // namespace fa
