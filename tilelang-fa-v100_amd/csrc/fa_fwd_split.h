// Dense attention forward for problems whose query tiles cannot fill the GPU
// (gfx950): keys split across the waves of a workgroup.
//
// Same mathematics as the other forward cores (the reference's
// _forward_lse_kernel_func, tilelang_fa_v100/_kernels_forward.py:94-172):
// online softmax over the visible keys, O = Σ P V / Σ P, LSE = m·scale + ln l.
// The 128- and 256-row cores give every wave 32 query rows and all of their
// keys, so a problem with few query tiles (the reference's configs[0],
// [1, 512, 16, 64]: 64 workgroups for 256 CUs) leaves most CUs idle and each
// wave's serial walk over the keys sets the time.  Here a workgroup owns 32
// query rows of one head and its NW waves split the keys those rows see
// into NW contiguous ranges (multiples of 32 keys):
//  * each wave copies its own 32-key K / V tiles HBM -> LDS
//    (global_load_lds_dwordx4, 16-byte chunks swizzled per row) into a
//    private double buffer, so the key loop needs no barrier;
//  * per tile, Sᵀ = K Qᵀ (the lane's scores all belong to its own query row),
//    mask, online softmax with a lazily rescaled running max, and
//    Oᵀ += Vᵀ Pᵀ with Vᵀ by ds_read_b64_tr_b16 and Pᵀ packed from the
//    accumulators;
//  * the waves' partial (O, running max, row sum) go to LDS and are merged per
//    row, O = Σ_w O_w 2^(m_w − M) / Σ_w l_w 2^(m_w − M), M = max_w m_w (the
//    merge the split-KV decode and prefill combines use).
#pragma once

#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

template <int D_>
struct FwdSplitShape {
  static constexpr int D = D_;
  static constexpr int NW = D == 64 ? tiles::kFwdSplitWaves64 : tiles::kFwdSplitWaves128;
  static constexpr int BK = 32;                  // keys per tile
  static constexpr int ROWB = 2 * D;             // bytes per K / V row
  static constexpr int CPR = D / 8;              // 16-byte chunks per row
  static constexpr int RPB = 1024 / ROWB;        // rows per 1 KB DMA block
  static constexpr int TILEB = BK * ROWB;        // one K or V tile
  static constexpr int BLKS = TILEB / 1024;      // DMA blocks per tile
  // Tile buffers per wave: two (the next tile's DMA under the current
  // tile's products) while they fit 128 KB of LDS in all, else one.
  static constexpr int NBUF = NW * 4 * TILEB <= 128 * 1024 ? 2 : 1;
  static constexpr int WAVEB = NBUF * 2 * TILEB;  // NBUF buffers of (K, V)
  // Merge area (reuses the tile buffers): O partial rows padded by 4 floats.
  static constexpr int OPS = D + 4;
  static constexpr int MERGE = NW * 32 * OPS * 4 + 2 * NW * 32 * 4;
  static constexpr int LDS = NW * WAVEB > MERGE ? NW * WAVEB : MERGE;
  static constexpr int SWZ = CPR >= 16 ? 15 : CPR - 1;  // chunk swizzle bits
  static_assert((D == 64 || D == 128) && BLKS * 1024 == TILEB, "shape");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert(32 % NW == 0 && 64 % (32 / NW) == 0 && D % (64 / (32 / NW)) == 0 &&
                    (D / (64 / (32 / NW))) % 2 == 0,
                "merge split");
};

template <class T, int D_, int MODE>
__global__ __launch_bounds__(64 * FwdSplitShape<D_>::NW) void fwd_split_kernel(fa_fwd_args a) {
  using S = FwdSplitShape<D_>;
  constexpr int D = S::D, NW = S::NW, ROWB = S::ROWB;
  __shared__ __attribute__((aligned(16))) char smem[S::LDS];
  constexpr float kLazy = 8.f;

  const int Sq = a.seqlen_q, Sk = a.seqlen_k, H = a.num_heads;
  const int nblk = (Sq + 31) / 32;
  const TileHead th = xcd_tile_order(blockIdx.x, nblk, a.batch * H);
  const int bh = th.bh, h = bh % H, b = bh / H;
  const int hk = h / (H / a.num_heads_k);
  const int row0 = 32 * th.rank;
  const Band band = mode_band<MODE>(a);
  auto kv_lo = [&](int r) { return band.wl >= 0 ? min(max(r + band.off - band.wl, 0), Sk) : 0; };
  auto kv_hi = [&](int r) {
    return band.wr >= 0 ? min(max(r + band.off + band.wr + 1, 0), Sk) : Sk;
  };

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  const float scale_log2 = a.softmax_scale * kLog2e;

  const int row_last = min(row0 + 31, Sq - 1);
  const int row = row0 + lr;
  const bool row_valid = row < Sq;
  const int my_lo = row_valid ? kv_lo(row) : 0, my_hi = row_valid ? kv_hi(row) : 0;
  // The keys any row of the block sees, [k_lo, k_hi), in NW ranges of whole
  // 32-key tiles; this wave's tiles are [t0, t1).
  const int k_lo = kv_lo(row0) / 32 * 32, k_hi = kv_hi(row_last);
  const int ntiles = max((k_hi - k_lo + 31) / 32, 0);
  const int per = (ntiles + NW - 1) / NW;
  const int t0 = min(wave * per, ntiles), t1 = min(t0 + per, ntiles);

  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[2];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[2];

  // ---- wave-private tiles: [buffer][K, V][32 rows][ROWB], chunk c of row r
  // stored at chunk c ^ swz(r).
  char* const wbase = smem + wave * S::WAVEB;
  auto kbuf = [&](int bf) { return wbase + bf * 2 * S::TILEB; };  // bf < NBUF
  auto vbuf = [&](int bf) { return wbase + bf * 2 * S::TILEB + S::TILEB; };
  auto swz = [](int r) { return swz_chunk(r) & S::SWZ; };
  // DMA of tile t (keys k_lo + 32t ..): lane l of block blk holds row
  // RPB blk + l / CPR, stored chunk l % CPR; rows past the last key repeat it
  // (their scores are masked).
  auto issue = [&](int t, int bf) {
    const int n0 = k_lo + 32 * t;
#pragma unroll
    for (int blk = 0; blk < S::BLKS; ++blk) {
      const int r = S::RPB * blk + lane / S::CPR;
      const int c = (lane % S::CPR) ^ swz(r);
      const int64_t n = min(n0 + r, Sk - 1);
      global_lds16_opaque(kg + n * a.k_stride[1] + 8 * c, kbuf(bf) + blk * 1024);
      global_lds16_opaque(vg + n * a.v_stride[1] + 8 * c, vbuf(bf) + blk * 1024);
    }
  };
  // K operand of Sᵀ = K Qᵀ, chunk c: row lr, logical chunk 2c + lh.
  int koff[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) koff[c] = lr * ROWB + 16 * ((2 * c + lh) ^ swz(lr));
  // Vᵀ operand, 16-key chunk kc, d tile dt: lane k reads 4 halves of row
  // 16kc + 4(k/32) + (k%16)/4 (+8 for the upper half), columns 32dt +
  // 16((k/16)%2) + 4(k%4).  The swizzle of row 16kc + x equals that of x.
  int voff[2][D / 32];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * hf;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      voff[hf][dt] = r * ROWB + 16 * (chunk ^ swz(r)) + 8 * (lane & 1);
    }
  }

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float ms_run = neg_inf(), l_run = 0.f;
  u32x4 qf[D / 16];  // the lane's query row (B operand chunks), loaded below

  auto compute = [&](int t, int bf) {
    const int n0 = k_lo + 32 * t;
    const char* kb = kbuf(bf);
    const char* vb = vbuf(bf);
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) s = T::mma32(ld16(kb + koff[c]), qf[c], s);
    // Element i is key n0 + 8(i/4) + 4lh + i%4 of the lane's row (rows past
    // Sq compute garbage that the merge never stores).
    if (n0 < kv_lo(row_last) || n0 + 32 > kv_hi(row0)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kv = n0 + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (kv < my_lo || kv >= my_hi) s[i] = neg_inf();
      }
    }
    float mt = neg_inf();
#pragma unroll
    for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[i]);
    mt = half_max(mt) * scale_log2;
    // The running max only moves when the tile's exceeds it by more than
    // kLazy (P <= 2^kLazy), so O is rescaled on few tiles.
    const bool grow = mt > ms_run + kLazy;
    if (__any(grow)) {
      const float ms_new = grow ? mt : ms_run;
      const float alpha = grow ? fast_exp2(ms_run - ms_new) : 1.f;
      ms_run = ms_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }
    const float mb = ms_run == neg_inf() ? 0.f : ms_run;
    u32x4 pb[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e = 8 * kc + 2 * w;
        const float p0 = fast_exp2(fmaf(s[e], scale_log2, -mb));
        const float p1 = fast_exp2(fmaf(s[e + 1], scale_log2, -mb));
        pb[kc][w] = T::pack(p0, p1);
        l_run = T::sum2(p0, p1, pb[kc][w], l_run);
      }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const u32x2 lo = lds_read_tr(vb + voff[0][dt] + kc * 16 * ROWB);
        const u32x2 hi = lds_read_tr(vb + voff[1][dt] + kc * 16 * ROWB);
        o[dt] = T::mma32(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb[kc], o[dt]);
      }
  };

  // ---- the wave's key loop: tile t in buffer (t - t0) % 2; the DMA of tile
  // t + 1 is in flight while tile t is computed (2 BLKS DMAs per tile).
  if (t0 < t1) issue(t0, 0);
  // The lane's query row as B operand chunks (zero for rows past Sq), loaded
  // while the first tile is in flight; one wait covers both, so the
  // compiler's own wait before the first product (it does not see the DMA)
  // cannot also wait for the next tile's.
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.q_stride[0] +
                         h * a.q_stride[2] + (int64_t)min(row, Sq - 1) * a.q_stride[1];
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      qf[c] = row_valid ? ld16(qp + 16 * c + 8 * lh) : u32x4{0, 0, 0, 0};
  }
  wait_vmem();
  for (int t = t0; t < t1; ++t) {
    const int bf = S::NBUF == 2 ? (t - t0) & 1 : 0;
    if (S::NBUF == 2 && t + 1 < t1) {
      issue(t + 1, bf ^ 1);
      if constexpr (2 * S::BLKS == 8)
        __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): tile t landed
      else
        __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16)
    } else {
      wait_vmem();
    }
    compute(t, bf);
    // The next DMA into this buffer is issued after the operand reads of
    // this tile have returned.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    if (S::NBUF == 1 && t + 1 < t1) issue(t + 1, 0);
  }

  // ---- merge.  Each wave's partial for its 32 rows: O (fp32, unnormalised
  // relative to 2^m), m = running max (base 2, scaled), l = row sum.
  const float l_all = half_sum(l_run);
  __syncthreads();  // every wave is done with its tile buffers
  float* op = reinterpret_cast<float*>(smem);  // [NW][32][OPS]
  float* mlp = op + NW * 32 * S::OPS;          // [NW][2][32]
  {
    float* orow = op + (wave * 32 + lr) * S::OPS;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(orow + 32 * dt + 8 * g + 4 * lh) =
            f32x4{o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]};
    if (lh == 0) {
      mlp[wave * 64 + lr] = ms_run;
      mlp[wave * 64 + 32 + lr] = l_all;
    }
  }
  __syncthreads();
  // Wave w merges rows RPW w .. RPW w + RPW - 1; LPR lanes per row, DPL
  // columns per lane.
  constexpr int RPW = 32 / NW, LPR = 64 / RPW, DPL = D / LPR;
  const int mr = RPW * wave + lane / LPR;
  const int d0 = DPL * (lane % LPR);
  const int orow_g = row0 + mr;
  float M = neg_inf();
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, mlp[w * 64 + mr]);
  float L = 0.f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
  if (M != neg_inf()) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = fast_exp2(mlp[w * 64 + mr] - M);  // 0 for an empty range
      L = fmaf(mlp[w * 64 + 32 + mr], f, L);
      const float* src = op + (w * 32 + mr) * S::OPS + d0;
#pragma unroll
      for (int j = 0; j < DPL; j += 2) {
        const float2 x = *reinterpret_cast<const float2*>(src + j);
        acc[j] = fmaf(x.x, f, acc[j]);
        acc[j + 1] = fmaf(x.y, f, acc[j + 1]);
      }
    }
  }
  if (orow_g >= Sq) return;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* dst = static_cast<uint16_t*>(a.out) + b * a.o_stride[0] + h * a.o_stride[2] +
                  (int64_t)orow_g * a.o_stride[1] + d0;
#pragma unroll
  for (int j = 0; j < DPL; j += 2)
    *reinterpret_cast<uint32_t*>(dst + j) = T::pack(acc[j] * inv, acc[j + 1] * inv);
  if (a.lse && lane % LPR == 0)
    a.lse[(int64_t)bh * Sq + orow_g] = L > 0.f ? (M + log2f(L)) * kLn2 : neg_inf();
}

}  // namespace fa
