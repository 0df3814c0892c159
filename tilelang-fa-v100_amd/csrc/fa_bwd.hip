// Dense attention backward for gfx950 (FlashAttention-2, LSE recompute).
//
// Replaces tilelang_backward (tilelang_fa_v100/_kernels_backward.py:200-208):
// the PyTorch row_dot (:203), the dQ kernel (:10-85) and the dK/dV kernel
// (:88-176).  The reference recomputes QK^T and dO V^T in both kernels (7
// GEMMs per tile pair); here one KV-stationary kernel does the 5 GEMMs
//   S = Q K^T,  dP = dO V^T,  dV += P^T dO,  dK += dS^T Q,  dQ += dS K
// with P = exp(scale*S - lse), dS = P * (dP - rowdot(O, dO)) * scale
// (_kernels_backward.py:72-74,159-170).  dQ comes from a query-stationary
// kernel (fa_bwd_dq.h) that recomputes S and dP per query tile and builds
// each dQ row in one wave, like the reference's dQ kernel: no atomics, so
// dq, dk and dv repeat bit for bit (fp32 atomics into a dQ accumulator were
// measured slower at every head_dim: they are performed beyond the XCD's L2
// on this part).
//
// Kernels, in launch order:
//   bwd_dq_kernel       dQ (fa_bwd_dq.h); also writes the row statistics
//                       scale·rowdot(O, dO) and LSE*log2(e) of the rows it
//                       owns into one array [B*H][2][Sq] (LSE*log2(e)
//                       first, scale·rowdot second), so a lane of the dK / dV
//                       kernels addresses either with a 32-bit offset from a
//                       per-head base.
// Every kernel forms dS already multiplied by softmax_scale and rounds that
// to 16 bits before its products, as the reference does
// (_kernels_backward.py:74,160), so dS has fp16's full range.
//   bwd_main_kernel     head_dim 64 dK / dV: workgroup = 128 keys (32 per
//                       wave) of one KV head; loops over the 64-row query
//                       tiles of every query head that shares the KV head
//                       (GQA).  K and V of the wave stay in registers.
//   bwd_main_mfma_kernel  head_dim 128 / 256 dK / dV (fa_bwd_mfma.h).
// At head_dim 128 / 256 with causal or full attention and a workspace of
// bwd_workspace_bytes, the order is instead bwd_stats_kernel (the row
// statistics), bwd_main_mfma_kernel<..., DS = true> (dK / dV, storing its dS
// tiles) and bwd_dq_ds_kernel (dQ = dS K from them), fa_bwd_ds.h.
#include "fa_bwd_dq.h"
#include "fa_bwd_ds.h"
#include "fa_bwd_mfma.h"
#include "fa_common.h"
#include "fa_internal.h"

namespace fa {

template <int D>
struct BwdShape {
  static constexpr int BKV = tiles::kBwd64Keys;       // keys per workgroup
  static constexpr int BQ = tiles::kBwd64QueryRows;   // query rows per iteration
  static constexpr int NQT = BQ / 32;     // 32-row query sub-tiles
  static constexpr int DC = D / 16;       // 16-wide d chunks (QK^T, dO V^T)
  static constexpr int DT = D / 32;       // 32-wide d tiles (dK^T, dV^T, dQ)
  static constexpr int CPR = D / 8;       // 16-byte chunks per row
  static constexpr int RG = BQ * CPR / 256;  // consecutive rows per thread
  static constexpr int QS = D + 8;        // natural Q / dO row stride
  static constexpr int TS = BQ + 4;       // transposed Q / dO row stride
  static constexpr int OFF_QS = 0;
  static constexpr int OFF_DOS = OFF_QS + BQ * QS;
  static constexpr int OFF_QT = OFF_DOS + BQ * QS;
  static constexpr int OFF_DOT = OFF_QT + D * TS;
  static constexpr int LDS_ELEMS = OFF_DOT + D * TS;
  static_assert(RG == 2 || RG == 4, "row grouping");
};

// ------------------------------------------------------------ main kernel
// head_dim 64: dK / dV only (dQ comes from bwd_dq_kernel).  MODE (MaskMode):
// full attention, causal, or a window band from the arguments.
template <class T, int D, int MODE>
__global__ __launch_bounds__(256, 2) void bwd_main_kernel(fa_bwd_args a, const float* stats) {
  using S = BwdShape<D>;
  constexpr bool CAUSAL = MODE != kMaskNone;  // some (query, key) pairs are outside the band
  __shared__ __attribute__((aligned(16))) uint16_t smem[S::LDS_ELEMS];
  __shared__ __attribute__((aligned(16))) float lse_s[S::BQ];
  __shared__ __attribute__((aligned(16))) float di_s[S::BQ];
  uint16_t* Qs = smem + S::OFF_QS;
  uint16_t* dOs = smem + S::OFF_DOS;
  uint16_t* Qt = smem + S::OFF_QT;
  uint16_t* dOt = smem + S::OFF_DOT;

  const int Sq = a.seqlen_q, Sk = a.seqlen_k, H = a.num_heads, Hk = a.num_heads_k;
  const int G = H / Hk;  // query heads sharing this KV head
  const int kvtiles = (Sk + S::BKV - 1) / S::BKV;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int kt_idx = id % kvtiles;  // smallest key index first: most query rows
  const int bh = id / kvtiles;
  const int hk = bh % Hk, b = bh / Hk;
  const int kv0 = kt_idx * S::BKV;
  const Band band = mode_band<MODE>(a);  // kMaskNone: no band (full attention)

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  const int kv0w = kv0 + 32 * wave;
  const int my_kv = kv0w + lr;
  const float scale_log2 = a.softmax_scale * kLog2e;
  const float sc = a.softmax_scale;

  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[2];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[2];

  // ---- stationary operands: K, V rows of this lane (B operands).
  u32x4 kB[S::DC], vB[S::DC];
  {
    const bool ok = my_kv < Sk;
    const uint16_t* kp = kg + (int64_t)my_kv * a.k_stride[1];
    const uint16_t* vp = vg + (int64_t)my_kv * a.v_stride[1];
#pragma unroll
    for (int c = 0; c < S::DC; ++c) {
      kB[c] = ok ? ld16(kp + 16 * c + 8 * lh) : u32x4{0, 0, 0, 0};
      vB[c] = ok ? ld16(vp + 16 * c + 8 * lh) : u32x4{0, 0, 0, 0};
    }
  }

  f32x16 dk[S::DT], dv[S::DT];
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) dk[dt][i] = dv[dt][i] = 0.f;

  // Query rows that can see any key of this tile.
  const int q_begin = CAUSAL ? band.first_row(kv0) : 0;
  const int q_end = CAUSAL ? band.end_row(kv0 + S::BKV - 1, Sq) : Sq;
  const int it0 = q_begin / S::BQ;
  const int it1 = (q_end + S::BQ - 1) / S::BQ;
  const int nit = max(it1 - it0, 0);
  const int wkv_last = min(kv0w + 31, Sk - 1);

  // Iteration t covers query head hk*G + t / nit, query tile it0 + t % nit.
  // Q / dO tile loader: thread owns column chunk col8 of RG consecutive rows.
  const int col8 = tid % S::CPR;
  const int rg0 = (tid / S::CPR) * S::RG;
  u32x4 qreg[S::RG], doreg[S::RG];
  float lreg = 0.f, dreg = 0.f;
  auto load_q = [&](int t) {
    const int h = hk * G + t / nit;
    const int i0 = (it0 + t % nit) * S::BQ;
    const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_stride[0] + h * a.q_stride[2];
    const uint16_t* dog = static_cast<const uint16_t*>(a.dout) + b * a.do_stride[0] +
                          h * a.do_stride[2];
    const int64_t stat0 = ((int64_t)b * H + h) * Sq;
#pragma unroll
    for (int r = 0; r < S::RG; ++r) {
      const int i = i0 + rg0 + r;
      const bool ok = i < Sq;
      qreg[r] = ok ? ld16(qg + (int64_t)i * a.q_stride[1] + 8 * col8) : u32x4{0, 0, 0, 0};
      doreg[r] = ok ? ld16(dog + (int64_t)i * a.do_stride[1] + 8 * col8) : u32x4{0, 0, 0, 0};
    }
    if (tid < S::BQ) {
      const int i = i0 + tid;
      lreg = i < Sq ? stats[2 * stat0 + i] : __builtin_inff();
      dreg = i < Sq ? stats[2 * stat0 + Sq + i] : 0.f;
    }
  };
  auto store_q = [&]() {
#pragma unroll
    for (int r = 0; r < S::RG; ++r) {
      st16(Qs + (rg0 + r) * S::QS + 8 * col8, qreg[r]);
      st16(dOs + (rg0 + r) * S::QS + 8 * col8, doreg[r]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int w = j >> 1;
      if constexpr (S::RG == 4) {
        u32x2 pq, pd;
        pq[0] = (j & 1) ? pack_hi(qreg[0][w], qreg[1][w]) : pack_lo(qreg[0][w], qreg[1][w]);
        pq[1] = (j & 1) ? pack_hi(qreg[2][w], qreg[3][w]) : pack_lo(qreg[2][w], qreg[3][w]);
        pd[0] = (j & 1) ? pack_hi(doreg[0][w], doreg[1][w]) : pack_lo(doreg[0][w], doreg[1][w]);
        pd[1] = (j & 1) ? pack_hi(doreg[2][w], doreg[3][w]) : pack_lo(doreg[2][w], doreg[3][w]);
        st8(Qt + (8 * col8 + j) * S::TS + rg0, pq);
        st8(dOt + (8 * col8 + j) * S::TS + rg0, pd);
      } else {
        const uint32_t pq = (j & 1) ? pack_hi(qreg[0][w], qreg[1][w]) : pack_lo(qreg[0][w], qreg[1][w]);
        const uint32_t pd = (j & 1) ? pack_hi(doreg[0][w], doreg[1][w]) : pack_lo(doreg[0][w], doreg[1][w]);
        *reinterpret_cast<uint32_t*>(Qt + (8 * col8 + j) * S::TS + rg0) = pq;
        *reinterpret_cast<uint32_t*>(dOt + (8 * col8 + j) * S::TS + rg0) = pd;
      }
    }
    if (tid < S::BQ) {
      lse_s[tid] = lreg;
      di_s[tid] = dreg;
    }
  };

  const int ntot = nit * G;
  if (ntot > 0) {
    load_q(0);
    store_q();
  }
  for (int t = 0; t < ntot; ++t) {
    const int i0 = (it0 + t % nit) * S::BQ;
    __syncthreads();  // Q/dO tile visible
    const bool more = t + 1 < ntot;
    if (more) load_q(t + 1);

    // Does this wave's key block see any of these query rows?
    const bool active = !CAUSAL || band.any(i0, i0 + S::BQ - 1, kv0w, kv0w + 31);
    const bool wvalid = kv0w < Sk;
    if (active && wvalid) {
      f32x16 s[S::NQT], dp[S::NQT];
#pragma unroll
      for (int qt = 0; qt < S::NQT; ++qt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[qt][i] = dp[qt][i] = 0.f;
#pragma unroll
        for (int c = 0; c < S::DC; ++c) {
          const u32x4 aq = ld16(Qs + (qt * 32 + lr) * S::QS + 16 * c + 8 * lh);
          const u32x4 ado = ld16(dOs + (qt * 32 + lr) * S::QS + 16 * c + 8 * lh);
          s[qt] = T::mma32(aq, kB[c], s[qt]);
          dp[qt] = T::mma32(ado, vB[c], dp[qt]);
        }
      }
      // Masking is needed on the diagonal band and on a partial key block.
      const bool need_mask = (CAUSAL && !band.all(i0, i0 + S::BQ - 1, kv0w, wkv_last)) ||
                             (kv0w + 32 > Sk);
#pragma unroll
      for (int qt = 0; qt < S::NQT; ++qt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int qb = qt * 32 + 8 * g + 4 * lh;  // first of 4 rows
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse_s + qb);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(di_s + qb);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 4 * g + r;
            float p = fast_exp2(fmaf(s[qt][i], scale_log2, -l4[r]));
            if (need_mask) {
              const int qi = i0 + qb + r;
              const bool vis = (my_kv < Sk) && (!CAUSAL || band.in(qi, my_kv));
              p = vis ? p : 0.f;
            }
            s[qt][i] = p;                       // P
            // scale·dS, rounded to 16 bits as the reference does
            // (_kernels_backward.py:160); d4 holds scale·rowdot.
            dp[qt][i] = p * fmaf(dp[qt][i], sc, -d4[r]);
          }
        }
      // Pack P and dS as B operands.
      u32x4 pB[2 * S::NQT], sB[2 * S::NQT];
#pragma unroll
      for (int kq = 0; kq < 2 * S::NQT; ++kq)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int e = 8 * (kq & 1) + 2 * w;
          pB[kq][w] = T::pack(s[kq >> 1][e], s[kq >> 1][e + 1]);
          sB[kq][w] = T::pack(dp[kq >> 1][e], dp[kq >> 1][e + 1]);
        }
      // dV^T += dO^T P,  dK^T += Q^T dS
#pragma unroll
      for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
        for (int kq = 0; kq < 2 * S::NQT; ++kq) {
          const int qo = 16 * kq + 4 * lh;
          const uint16_t* tq = Qt + (dt * 32 + lr) * S::TS + qo;
          const uint16_t* td = dOt + (dt * 32 + lr) * S::TS + qo;
          const u32x2 q0 = ld8(tq), q1 = ld8(tq + 8);
          const u32x2 d0 = ld8(td), d1 = ld8(td + 8);
          const u32x4 aq = {q0[0], q0[1], q1[0], q1[1]};
          const u32x4 ad = {d0[0], d0[1], d1[0], d1[1]};
          dv[dt] = T::mma32(ad, pB[kq], dv[dt]);
          dk[dt] = T::mma32(aq, sB[kq], dk[dt]);
        }
    }
    __syncthreads();  // Q/dO tiles no longer read
    if (more) store_q();
  }

  // ---- epilogue: this lane's key row.
  if (my_kv < Sk) {
    uint16_t* dkp = static_cast<uint16_t*>(a.dk) + b * a.dk_stride[0] +
                    (int64_t)my_kv * a.dk_stride[1] + hk * a.dk_stride[2];
    uint16_t* dvp = static_cast<uint16_t*>(a.dv) + b * a.dv_stride[0] +
                    (int64_t)my_kv * a.dv_stride[1] + hk * a.dv_stride[2];
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * lh;
        u32x2 wk, wv;
        wk[0] = T::pack(dk[dt][4 * g], dk[dt][4 * g + 1]);
        wk[1] = T::pack(dk[dt][4 * g + 2], dk[dt][4 * g + 3]);
        wv[0] = T::pack(dv[dt][4 * g], dv[dt][4 * g + 1]);
        wv[1] = T::pack(dv[dt][4 * g + 2], dv[dt][4 * g + 3]);
        st8(dkp + d, wk);
        st8(dvp + d, wv);
      }
  }
}

// ----------------------------------------------------------------- launchers

// Workspace: the row statistics [B*H][2][Sq] (LSE*log2(e), scale·rowdot), then,
// for the dS-store path, the dS tiles (fa_bwd_ds.h) from byte ds_offset(a).
static size_t stats_bytes(const fa_bwd_args& a) {
  const size_t rows = (size_t)a.batch * a.seqlen_q * a.num_heads;
  return 2 * rows * sizeof(float) + 256;
}
static size_t ds_offset(const fa_bwd_args& a) { return (stats_bytes(a) + 255) & ~(size_t)255; }

// Bytes of dS tiles for the dS-store path, or 0 where it does not apply:
// head_dim 128 / 256, causal or full attention, below tiles::kBwdDsMaxBytes.
static size_t ds_bytes(const fa_bwd_args& a) {
  const int mode = mask_mode(a);
  if ((a.head_dim != 128 && a.head_dim != 256) || mode == kMaskBand || a.seqlen_q <= 0 ||
      a.seqlen_k <= 0)
    return 0;
  const DsTiles L = mode == kMaskCausal ? ds_tiles<kMaskCausal>(a.seqlen_q, a.seqlen_k)
                                        : ds_tiles<kMaskNone>(a.seqlen_q, a.seqlen_k);
  const size_t bytes = 2048 * (size_t)a.batch * a.num_heads * (size_t)L.per_head();
  // Strictly below the cap: a wave's dS reads go through one buffer resource
  // of count(qt) * 2 KB bytes (a 32-bit size), and count(qt) <= per_head.
  return bytes < tiles::kBwdDsMaxBytes ? bytes : 0;
}

size_t bwd_min_workspace_bytes(const fa_bwd_args& a) { return stats_bytes(a); }

size_t bwd_workspace_bytes(const fa_bwd_args& a) {
  const size_t ds = ds_bytes(a);
  return ds ? ds_offset(a) + ds : stats_bytes(a);
}

// Key-stationary dK / dV kernel for one mask mode; with ds, also stores the
// dS tiles (head_dim 128 / 256, causal or full attention).
template <class T, int D>
static void launch_bwd_main(const fa_bwd_args& a, int mode, const float* stats, uint16_t* ds,
                            hipStream_t st) {
  if constexpr (D >= 128) {
    using S = BwdShapeMfma<D>;
    const int kvtiles = (a.seqlen_k + S::BKV - 1) / S::BKV;
    const dim3 grid((unsigned)kvtiles * a.num_heads_k * a.batch), block(64 * S::NW);
    if (kvtiles == 0) return;  // no keys: dK / dV are empty
    {
      if (ds) {
        if (mode == kMaskCausal)
          hipLaunchKernelGGL((bwd_main_mfma_kernel<T, D, kMaskCausal, true>), grid, block, 0, st,
                             a, stats, ds);
        else
          hipLaunchKernelGGL((bwd_main_mfma_kernel<T, D, kMaskNone, true>), grid, block, 0, st, a,
                             stats, ds);
        return;
      }
    }
    if (mode == kMaskCausal)
      hipLaunchKernelGGL((bwd_main_mfma_kernel<T, D, kMaskCausal>), grid, block, 0, st, a, stats,
                         nullptr);
    else if (mode == kMaskBand)
      hipLaunchKernelGGL((bwd_main_mfma_kernel<T, D, kMaskBand>), grid, block, 0, st, a, stats,
                         nullptr);
    else
      hipLaunchKernelGGL((bwd_main_mfma_kernel<T, D, kMaskNone>), grid, block, 0, st, a, stats,
                         nullptr);
  } else {
    using S = BwdShape<D>;
    const int kvtiles = (a.seqlen_k + S::BKV - 1) / S::BKV;
    const dim3 grid((unsigned)kvtiles * a.num_heads_k * a.batch);
    if (kvtiles == 0) return;
    if (mode == kMaskCausal)
      hipLaunchKernelGGL((bwd_main_kernel<T, D, kMaskCausal>), grid, dim3(256), 0, st, a, stats);
    else if (mode == kMaskBand)
      hipLaunchKernelGGL((bwd_main_kernel<T, D, kMaskBand>), grid, dim3(256), 0, st, a, stats);
    else
      hipLaunchKernelGGL((bwd_main_kernel<T, D, kMaskNone>), grid, dim3(256), 0, st, a, stats);
  }
}

// Query-stationary dQ kernel (also writes the row statistics).
template <class T, int D>
static void launch_bwd_dq(const fa_bwd_args& a, int mode, float* stats, hipStream_t st) {
  using S = BwdDqShape<D>;
  const int qtiles = (a.seqlen_q + S::BM - 1) / S::BM;
  const dim3 grid((unsigned)qtiles * a.num_heads * a.batch), block(64 * S::NW);
  if (mode == kMaskCausal)
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kMaskCausal>), grid, block, 0, st, a, stats);
  else if (mode == kMaskBand)
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kMaskBand>), grid, block, 0, st, a, stats);
  else
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kMaskNone>), grid, block, 0, st, a, stats);
}

// dS-store path (head_dim 128 / 256): row statistics, dK / dV storing dS,
// then dQ = dS K (dS includes the scale).
template <class T, int D>
static hipError_t launch_bwd_ds(const fa_bwd_args& a, int mode, void* ws, hipStream_t st) {
  float* stats = static_cast<float*>(ws);
  uint16_t* ds = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + ds_offset(a));
  const int64_t blocks = (int64_t)a.batch * a.num_heads * ((a.seqlen_q + 31) / 32);
  constexpr int per_wg = 4 * StatsShape<D>::kTiles;  // 32-row blocks per workgroup
  hipLaunchKernelGGL((bwd_stats_kernel<T, D>), dim3((unsigned)((blocks + per_wg - 1) / per_wg)),
                     dim3(256), 0, st, a, stats);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_bwd_main<T, D>(a, mode, stats, ds, st);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  constexpr int NW = DqDsShape<D>::NW;
  const int nqb = ((a.seqlen_q + 31) / 32 + NW - 1) / NW;
  const dim3 grid((unsigned)nqb * a.num_heads * a.batch), block(64 * NW);
  if (mode == kMaskCausal)
    hipLaunchKernelGGL((bwd_dq_ds_kernel<T, D, kMaskCausal>), grid, block, 0, st, a, ds);
  else
    hipLaunchKernelGGL((bwd_dq_ds_kernel<T, D, kMaskNone>), grid, block, 0, st, a, ds);
  return hipGetLastError();
}

// dQ (and the row statistics), then dK / dV.  Every output element is
// produced by one fixed sequence of operations.  A workspace of
// bwd_workspace_bytes selects the dS-store path where it applies; one of
// bwd_min_workspace_bytes, the recompute path.
template <class T, int D>
static hipError_t launch_bwd_d(const fa_bwd_args& a, void* ws, size_t ws_bytes, hipStream_t st) {
  const int mode = mask_mode(a);
  if constexpr (D >= 128) {
    if (ds_bytes(a) && ws_bytes >= bwd_workspace_bytes(a)) return launch_bwd_ds<T, D>(a, mode, ws, st);
  }
  float* stats = static_cast<float*>(ws);  // [B*H][2][Sq]
  launch_bwd_dq<T, D>(a, mode, stats, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_bwd_main<T, D>(a, mode, stats, nullptr, st);
  return hipGetLastError();
}

template <class T>
static hipError_t launch_bwd_t(const fa_bwd_args& a, void* ws, size_t ws_bytes, hipStream_t st) {
  switch (a.head_dim) {
    case 64: return launch_bwd_d<T, 64>(a, ws, ws_bytes, st);
    case 128: return launch_bwd_d<T, 128>(a, ws, ws_bytes, st);
    case 256: return launch_bwd_d<T, 256>(a, ws, ws_bytes, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_bwd(const fa_bwd_args& a, void* ws, size_t ws_bytes, hipStream_t st) {
  return a.dtype == FA_DTYPE_BF16 ? launch_bwd_t<BFloat16>(a, ws, ws_bytes, st)
                                  : launch_bwd_t<Half>(a, ws, ws_bytes, st);
}

}  // namespace fa
