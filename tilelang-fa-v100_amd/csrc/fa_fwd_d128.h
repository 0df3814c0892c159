// Attention forward tile for head_dim 128 on gfx950: direct HBM->LDS tiles.
//
// Same algorithm and row-problem interface as attn_fwd_tile (fa_fwd_core.h),
// arranged for gfx950's memory instructions:
//  * 8 waves x 32 query rows (256 rows per workgroup), so every K/V tile in
//    LDS feeds twice as many MFMAs as a 4-wave tile.
//  * K and V tiles (64 keys x 256 B) go from HBM straight into LDS with
//    global_load_lds_dwordx4 (lane l of a wave writes bytes 16l..16l+15 of a
//    1 KB block): no staging registers, no VALU, no ds_write.  Each wave
//    loads 2 blocks (8 rows) of K and of V per tile, two tiles in flight.
//  * Both tiles stay row-major.  Vᵀ for Oᵀ = Vᵀ Pᵀ comes from
//    ds_read_b64_tr_b16, whose result for lane 16g+i, element j is element
//    i%4 of the 8 bytes addressed by lane 16g+4j+i/4.
//  * 16-byte chunk c of row r is stored at chunk c ^ swz(r) with
//    swz(r) = ((r & 3) << 2) | ((r >> 2) & 3).  The K operand read (16 rows
//    at one chunk per 16 lanes) and the transposed V read (4 rows x 4
//    consecutive chunks per 32 lanes) then touch 16 distinct chunk columns,
//    i.e. all 64 banks once.
//  * Every LDS address is precomputed per lane; tile and buffer offsets are
//    instruction immediates.
#pragma once

#include "fa_common.h"

namespace fa {

struct FwdShapeD128 {
  static constexpr int D = 128;
  static constexpr int BM = 256;          // query rows per workgroup
  static constexpr int BN = 64;           // keys per tile
  static constexpr int NW = 8;            // waves
  static constexpr int ROWB = 256;        // bytes per K/V row
  static constexpr int TILEB = BN * ROWB; // 16 KB per K or V tile
  static constexpr int LDS_BYTES = 2 * 2 * TILEB;  // 2 buffers x (K, V)
  static constexpr int LDS_ARRAY_BYTES = TILEB;    // each of the 4 arrays
};

__device__ __forceinline__ int swz_chunk(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));

__device__ __forceinline__ u32x2 lds_read_tr(const char* p) {
  auto lp = (__attribute__((address_space(3))) s16x4*)(p);
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(lp));
}

__device__ __forceinline__ void load_lds16(const void* g, char* lds_block) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_block, 16, 0, 0);
}

// Waits for this wave's outstanding global loads (including those that
// write LDS directly): vmcnt(0), expcnt/lgkmcnt untouched.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// k0/v0 and k1/v1 are four distinct __shared__ arrays of TILEB bytes.  The
// loop is unrolled by two so that every LDS read names one array pair while
// the DMA of the next tile targets the other; the compiler can then see that
// the reads do not depend on the outstanding DMA and does not wait for it.
template <class T, class Prob>
__device__ __forceinline__ void attn_fwd_tile_d128(const Prob& P, int row0, float scale,
                                                   char* k0, char* v0, char* k1, char* v1) {
  using S = FwdShapeD128;
  constexpr int D = S::D, BN = S::BN;
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

  // ---- per-lane LDS offsets (bytes, relative to a K or V tile base)
  // K operand of Sᵀ = K Qᵀ, chunk c: row lr (+32 kt), logical chunk 2c + lh.
  int koff[D / 16];
  {
    const int sw = swz_chunk(lr);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) koff[c] = lr * S::ROWB + 16 * ((2 * c + lh) ^ sw);
  }
  // Vᵀ operand, 16-key chunk kc, d tile dt: lane k reads 4 halves of row
  // 16kc + 4(k/32) + (k%16)/4 (+8 for the upper half), columns
  // 32dt + 16((k/16)%2) + 4(k%4).  The row's swizzle does not depend on kc.
  int voff[2][D / 32];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * hf;
    const int sw = swz_chunk(r);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      voff[hf][dt] = r * S::ROWB + 16 * (chunk ^ sw) + 8 * (lane & 1);
    }
  }

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float ms_run = neg_inf();
  float l_run = 0.f;

  // ---- tile loader: wave w fills 1 KB blocks 2w, 2w+1 (rows 8w .. 8w+7) of
  // the K and V tiles.  Lane l of block b holds row 4b + l/16, stored chunk
  // l%16, i.e. logical chunk (l%16) ^ swz(row).
  const int ld_last = max(wg_hi - 1, 0);
  auto issue_tile = [&](int n0, char* kb, char* vb) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int blk = 2 * wave + ii;
      const int r = 4 * blk + (lane >> 4);
      const int c = (lane & 15) ^ swz_chunk(r);
      const int n = min(n0 + r, ld_last);
      load_lds16(P.k_ptr(n) + 8 * c, kb + blk * 1024);
      load_lds16(P.v_ptr(n) + 8 * c, vb + blk * 1024);
    }
  };

  auto compute_tile = [&](int n0, const char* kb, const char* vb) {
    if (!(wave_active && n0 < w_hi_max && n0 + BN > w_lo_min)) return;
    f32x16 s[BN / 32];
#pragma unroll
    for (int kt = 0; kt < BN / 32; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kt][i] = 0.f;
    // The key blocks' accumulation chains alternate (consecutive products are
    // independent) and K reads run two chunks ahead of the products.
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int kt = 0; kt < BN / 32; ++kt)
        s[kt] = T::mma32(ld16(kb + koff[c] + kt * 32 * S::ROWB), qf[c], s[kt]);
    sched_pipeline<D / 16, BN / 32, BN / 32, 2>();
    const bool need_mask = (n0 < w_lo_max) || (n0 + BN > w_hi_min);
    if (need_mask) {
#pragma unroll
      for (int kt = 0; kt < BN / 32; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = n0 + kt * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
          if (kv < my_lo || kv >= my_hi) s[kt][i] = neg_inf();
        }
    }
    float mt = neg_inf();
#pragma unroll
    for (int kt = 0; kt < BN / 32; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[kt][i]);
    mt = fmaxf(mt, swap_halves(mt)) * scale_log2;
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
    u32x4 pb[BN / 16];
#pragma unroll
    for (int kc = 0; kc < BN / 16; ++kc)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e = 8 * (kc & 1) + 2 * w;
        const float p0 = fast_exp2(fmaf(s[kc >> 1][e], scale_log2, -mb));
        const float p1 = fast_exp2(fmaf(s[kc >> 1][e + 1], scale_log2, -mb));
        pb[kc][w] = T::pack(p0, p1);
        l_run = T::sum2(p0, p1, pb[kc][w], l_run);
      }
#pragma unroll
    for (int kc = 0; kc < BN / 16; ++kc)
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const u32x2 lo = lds_read_tr(vb + voff[0][dt] + kc * 16 * S::ROWB);
        const u32x2 hi = lds_read_tr(vb + voff[1][dt] + kc * 16 * S::ROWB);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        o[dt] = T::mma32(a, pb[kc], o[dt]);
      }
  };

  const int j0 = max(wg_lo, 0) / BN;
  const int j1 = (wg_hi + BN - 1) / BN;
  if (j0 < j1) issue_tile(j0 * BN, k0, v0);
  for (int j = j0; j < j1; j += 2) {
    // tile j in (k0, v0)
    wait_vmem();
    __syncthreads();  // tile j resident; everyone is done with tile j-1
    if (j + 1 < j1) issue_tile((j + 1) * BN, k1, v1);
    compute_tile(j * BN, k0, v0);
    if (j + 1 >= j1) break;
    // tile j+1 in (k1, v1)
    wait_vmem();
    __syncthreads();
    if (j + 2 < j1) issue_tile((j + 2) * BN, k0, v0);
    compute_tile((j + 1) * BN, k1, v1);
  }

  const float l_all = l_run + swap_halves(l_run);
  if (!row_valid) return;
  const float inv = l_all > 0.f ? 1.f / l_all : 0.f;
  uint16_t* op = P.o_ptr(row);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w[0] = T::pack(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv);
      w[1] = T::pack(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
      st8(op + 32 * dt + 8 * g + 4 * lh, w);
    }
  if (P.has_lse && lh == 0)
    *P.lse_ptr(row) = l_all > 0.f ? (ms_run + log2f(l_all)) * kLn2 : neg_inf();
}

}  // namespace fa
