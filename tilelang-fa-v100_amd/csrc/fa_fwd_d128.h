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
//  * Two schedules: attn_fwd_tile_d128 (two wave groups in alternating
//    matrix / softmax phases; dense problems and paged problems whose pages
//    hold at least 16 keys) and attn_fwd_tile_d128_plain (all waves in the
//    same phase, one barrier per tile; paged problems with smaller pages).
#pragma once

#include "fa_common.h"

namespace fa {

struct FwdShapeD128 {
  static constexpr int D = 128;
  static constexpr int BM = tiles::kFwd128Rows;   // query rows per workgroup
  static constexpr int BN = tiles::kFwd128Keys;   // keys per tile
  static constexpr int NW = tiles::kFwd128Waves;  // waves
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

// Waits for this wave's outstanding global loads (including those that
// write LDS directly): vmcnt(0), expcnt/lgkmcnt untouched.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// One-phase schedule (all waves score, exponentiate and accumulate the same
// tile between two barriers), used for paged problems whose pages hold fewer
// than 16 keys: their K / V rows need a block-table read each (the ping-pong
// schedule below takes 16-key runs at a fixed stride).
// k0/v0 and k1/v1 are four distinct __shared__ arrays of TILEB bytes.  The
// loop is unrolled by two so that every LDS read names one array pair while
// the DMA of the next tile targets the other; the compiler can then see that
// the reads do not depend on the outstanding DMA and does not wait for it.
template <class T, class Prob>
__device__ __forceinline__ void attn_fwd_tile_d128_plain(const Prob& P, int row0, float scale,
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
      global_lds16_opaque(P.k_ptr(n) + 8 * c, kb + blk * 1024);
      global_lds16_opaque(P.v_ptr(n) + 8 * c, vb + blk * 1024);
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
    mt = half_max(mt) * scale_log2;
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

  const float l_all = half_sum(l_run);
  if (!row_valid) return;
  fwd_store_row<T>(P, row, lh, o, l_all, ms_run);
}


// Ping-pong schedule, used for row-strided (dense) problems.
// k0/v0 and k1/v1 are four distinct __shared__ arrays of TILEB bytes.  The
// loop is unrolled by two so that every LDS read names one array pair while
// the DMA of the next tile targets the other; the compiler can then see that
// the reads do not depend on the outstanding DMA and does not wait for it.
//
// attn_fwd_tiles_d128 runs a sequence of row tiles on one workgroup:
// next(P, row0) rewrites the problem and first row for the next tile and
// returns false after the last one.  Between tiles no CU time is lost to a
// workgroup's teardown and launch: once every wave is past a tile's last
// barrier (LDS and the Q registers are free), the tile's output stores go
// out, then the next tile's Q rows and first K tile are requested, and their
// latencies overlap.
template <class T, class Prob, class Next>
__device__ __forceinline__ void attn_fwd_tiles_d128(Prob P, int row0, float scale, char* k0,
                                                    char* v0, char* k1, char* v1, Next next) {
  using S = FwdShapeD128;
  constexpr int D = S::D, BN = S::BN;
  const float scale_log2 = scale * kLog2e;
  constexpr float kLazy = 8.f;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  const bool grp_b = wave >= S::NW / 2;
  constexpr int DB = 16 / (S::NW / 2);  // blocks per DMA wave
  static_assert(DB * 4 == 16, "each DMA wave fills 16 rows");

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

  // K / V rows are a base plus a row stride: tiles are DMA'd through buffer
  // resources, the lane's byte offset within the tile is fixed, the tile
  // base is scalar, and rows at or past the last key read as zero (their
  // scores are masked).  Group A alone issues them, from inside its matrix
  // phase: issuing 32 KB per tile from all eight waves at the start of a
  // slot stalled them on the vector-memory queue; behind a burst of MFMAs
  // the queueing overlaps the matrix core's work (wave w < 4 fills 1 KB
  // blocks 4w .. 4w+3, i.e. keys n0 + 16w .. n0 + 16w + 15).  A wave's 16
  // rows are a base plus the row stride: for paged K / V (pages of at least
  // 16 keys) they lie in one page, whose block-table entry is one scalar
  // load per wave and tile.  The row strides are those of the launch, the
  // same for every tile.
  uint32_t k_loff[DB], v_loff[DB];
#pragma unroll
  for (int ii = 0; ii < DB; ++ii) {
    const int r = 4 * (DB * wave + ii) + (lane >> 4);  // row of the tile
    const uint32_t r16 = 4 * ii + (lane >> 4);         // row of the wave's 16
    const uint32_t chunk = 8u * ((lane & 15) ^ swz_chunk(r));
    k_loff[ii] = 2u * (r16 * (uint32_t)P.k_row_stride() + chunk);
    v_loff[ii] = 2u * (r16 * (uint32_t)P.v_row_stride() + chunk);
  }
  // Keys n0 .. n0 + 63 of the problem (keys below wg_hi exist) into dst.
  auto issue_rows = [&](int wg_hi, int n0, char* dst, auto is_v) {
    constexpr bool kV = decltype(is_v)::value;
    const int nw = n0 + 16 * wave;
    const int nvalid = min(16, wg_hi - nw);  // n0 < wg_hi, so n0's row resolves
    const int nb = nvalid > 0 ? nw : n0;
    const uint16_t* base = kV ? P.v_ptr(nb) : P.k_ptr(nb);
    // The range ends after the last valid row's D columns (not nvalid whole
    // strides): a size-1 sequence dimension may come with stride 0.
    const uint32_t bytes = span_bytes(nvalid, kV ? P.v_row_stride() : P.k_row_stride(), D);
    u32x4 rs = rsrc_words(base, bytes);
    // Uniform by construction (the block-table read of a paged problem is
    // not known to be); the resource must sit in scalar registers.
#pragma unroll
    for (int w = 0; w < 4; ++w) rs[w] = __builtin_amdgcn_readfirstlane(rs[w]);
    // (T1 forward 0.525 -> 0.513 ms, C3 paged prefill 0.546 -> 0.529 ms
    // against four single DMAs, same box.)
    static_assert(DB == 4, "four 1 KB blocks per DMA wave");
    const uint32_t* lo = kV ? v_loff : k_loff;
    buffer_lds16_x4(rs, lo[0], lo[1], lo[2], lo[3], dst + DB * wave * 1024);
  };

  // This lane's Q row of the tile (P, row0), and (group A) its first K tile
  // into k0.
  u32x4 qf[D / 16];
  auto start_tile = [&]() {
    // The lane index is formed afresh (an opaque v_mbcnt pair): held from
    // the kernel's start, its 8 * lh offset was the one VGPR value the dense
    // core spilled, and the reload's vmcnt(0) made the next tile's Q loads
    // wait for the previous tile's output stores (S1k / S2k forward -1.2% to
    // -1.8% without it, same box).
    uint32_t ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int rw = row0 + wave * 32 + (int)(ln & 31);
    const bool valid = rw < P.nrows;
    const uint16_t* qp = valid ? P.q_ptr(rw) + 8 * (int)(ln >> 5) : nullptr;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = valid ? ld16(qp + 16 * c) : u32x4{0, 0, 0, 0};
    const int hi = P.kv_hi(min(row0 + S::BM, P.nrows) - 1);
    const int lo = max(P.kv_lo(row0), 0) / BN * BN;
    if (lo < hi && !grp_b) issue_rows(hi, lo, k0, BoolC<false>{});
  };
  start_tile();

  for (;;) {

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
  // Paged problems: the row's output pointers are formed here and held in
  // VGPRs, so the arguments they come from (pointers, token and head
  // strides) are not live through the key loop, where they spilled from
  // the scalar registers (44 spilled SGPRs against 13; C3 paged prefill
  // 0.5195 / 0.5149 -> 0.5135 / 0.5127 ms, C5 -0.5%, same box).  The dense
  // core has no VGPRs to spare and forms them at the store.
  constexpr bool kEarlyOut = !Prob::kRowStrided;
  decltype(fwd_out_ptr(P, 0)) out_row = nullptr;
  float* lse_row = nullptr;
  if constexpr (kEarlyOut) {
    if (row_valid) {
      out_row = fwd_out_ptr(P, row);
      lse_row = fwd_lse_ptr(P, row);
    }
    asm volatile("" : "+v"(out_row), "+v"(lse_row));
  }

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float ms_run = neg_inf();
  float l_run = 0.f;

  // Tile n0 has keys this wave's rows see.
  auto visible = [&](int n0) { return wave_active && n0 < w_hi_max && n0 + BN > w_lo_min; };
  f32x16 s[BN / 32];
  u32x4 pb[BN / 16];
  // Operand reads run kAheadS / kAheadO steps ahead of the products.
#ifndef FA_FWD_AHEAD_S
#define FA_FWD_AHEAD_S 3
#endif
#ifndef FA_FWD_AHEAD_O
#define FA_FWD_AHEAD_O 4
#endif
  constexpr int kAheadS = FA_FWD_AHEAD_S, kAheadO = FA_FWD_AHEAD_O;
  // Sᵀ = K Qᵀ for tile n0 (keys from kb).  The key blocks' accumulation
  // chains alternate (consecutive products are independent).
  auto gemm_s = [&](const char* kb) {
#pragma unroll
    for (int kt = 0; kt < BN / 32; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kt][i] = 0.f;
    struct KOps {
      u32x4 k[BN / 32];
    };
    lds_pipeline<D / 16, kAheadS>(
        [&](int c) {
          KOps r;
#pragma unroll
          for (int kt = 0; kt < BN / 32; ++kt) r.k[kt] = ld16(kb + koff[c] + kt * 32 * S::ROWB);
          return r;
        },
        [&](int c, const KOps& r) {
#pragma unroll
          for (int kt = 0; kt < BN / 32; ++kt) s[kt] = T::mma32(r.k[kt], qf[c], s[kt]);
        });
  };
  // Online softmax of s (tile n0) into the B operand pb of Oᵀ += Vᵀ Pᵀ.
  auto softmax = [&](int n0) {
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
    // Optimistic pass (every row has a running max): exponentials against
    // the running max, without the row maximum (16 v_max3, whose issue slows
    // next to the partner's products, and a cross-lane step).  Kept when no
    // row of the wave gained 128 or more in its sum: then no P reached 2^8,
    // so no running max would have moved under the lazy rule below, and the
    // result is the one that rule gives, bit for bit (a P above 2^8 adds at
    // least ~255.99 to a sum whose own rounding stays far below 128).
    // Otherwise the pass is redone below from the scores.  T1 forward -2.8%,
    // full attention -1.7%, C2 -0.9%, paged prefill unchanged (same box).
    if (!__any(ms_run == neg_inf())) {
      float l_new = l_run;
#pragma unroll
      for (int kc = 0; kc < BN / 16; ++kc)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int e = 8 * (kc & 1) + 2 * w;
          const float p0 = fast_exp2(fmaf(s[kc >> 1][e], scale_log2, -ms_run));
          const float p1 = fast_exp2(fmaf(s[kc >> 1][e + 1], scale_log2, -ms_run));
          pb[kc][w] = T::pack(p0, p1);
          l_new = l_new + (p0 + p1);
        }
      // NaN scores fail the test and take the full pass.
      if (!__any(!(half_sum(l_new - l_run) < 128.f))) {
        l_run = l_new;
        return;
      }
    }
    float mt = neg_inf();
#pragma unroll
    for (int kt = 0; kt < BN / 32; ++kt)
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
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }
    const float mb = ms_run == neg_inf() ? 0.f : ms_run;
#pragma unroll
    for (int kc = 0; kc < BN / 16; ++kc)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e = 8 * (kc & 1) + 2 * w;
        const float p0 = fast_exp2(fmaf(s[kc >> 1][e], scale_log2, -mb));
        const float p1 = fast_exp2(fmaf(s[kc >> 1][e + 1], scale_log2, -mb));
        pb[kc][w] = T::pack(p0, p1);
        // The fp32 values, as the reference sums its fp32 scores
        // (_kernels_forward.py:150-152).  The one-instruction fp16 form
        // (T::sum2: v_dot2 of the packed pair) overlaps the partner wave's
        // matrix products worse: T1 forward 0.545 -> 0.521 ms with the two
        // adds (same box); a two-wave microbenchmark (one wave's MFMAs, the
        // other's softmax instruction mix) shows the same.
        l_run = l_run + (p0 + p1);
      }
  };
  // Oᵀ += Vᵀ Pᵀ (V from vb).
  auto gemm_o = [&](const char* vb) {
    struct VOps {
      u32x2 lo, hi;
    };
    lds_pipeline<(BN / 16) * (D / 32), kAheadO>(
        [&](int k) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          return VOps{lds_read_tr(vb + voff[0][dt] + kc * 16 * S::ROWB),
                      lds_read_tr(vb + voff[1][dt] + kc * 16 * S::ROWB)};
        },
        [&](int k, const VOps& r) {
          const int kc = k / (D / 32), dt = k % (D / 32);
          const u32x4 a = {r.lo[0], r.lo[1], r.hi[0], r.hi[1]};
          o[dt] = T::mma32(a, pb[kc], o[dt]);
        });
  };

  // Ping-pong schedule.  Waves 0-3 (group A) and 4-7 (group B) share the
  // SIMDs pairwise; between two workgroup barriers (one per tile) each wave
  // runs two phases in opposite order to its partner, so one wave of each
  // SIMD runs matrix products (Oᵀ of the previous tile, then Sᵀ of the
  // current one: 32 MFMAs) while the other runs the softmax (exp2, max,
  // sums: VALU), instead of both waves reaching the same phase together.
  // Group B runs one phase behind group A (a barrier between the two phases
  // as well measured 2% slower):
  //   period j:  A: O(j-1), S(j), DMA K(j+1), V(j); then softmax(j)
  //              B: softmax(j-1); then O(j-1), S(j)
  //              wait for the DMA, barrier
  // K(j) is read in period j and V(j) in period j+1, so two buffers of each
  // suffice: K(j+1) and V(j) overwrite K(j-1) and V(j-2), whose last reads
  // were in period j-1, before its barrier.  The loop body covers two tiles
  // so that every buffer is a compile-time array (see the note on k0..v1
  // above).
  const int j0 = max(wg_lo, 0) / BN;
  const int j1 = (wg_hi + BN - 1) / BN;
  auto issue_k = [&](int n0, char* kb) { issue_rows(wg_hi, n0, kb, BoolC<false>{}); };
  auto issue_v = [&](int n0, char* vb) { issue_rows(wg_hi, n0, vb, BoolC<true>{}); };
  // One slot: the matrix phase for tile j (O of j-1 from vprev, S of j from
  // kcur; group A also issues the DMA of K(j+1) into knext and V(j) into
  // vcur) or the softmax phase for tile js.
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
  // Wait for this wave's DMA, then the workgroup barrier that makes every
  // wave's DMA visible and frees the buffers read before it.
  auto tile_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  // The tile's Q rows and first K tile (start_tile) have landed.
  wait_vmem();
  __syncthreads();
  // Each group runs its own copy of the loop (the barriers pair up across
  // the copies: both execute the same number), so that in each copy only
  // one of s / pb is live at a slot boundary.
  auto run = [&](auto group_b) {
    constexpr bool kB = decltype(group_b)::value;
    constexpr BoolC<!kB> dma{};
    for (int j = j0;; j += 2) {
      // tile j: K in k0, V in v0; tile j-1: V in v1; tile j+1: K in k1.
      if (kB) sm_phase(j - 1); else mma_phase(j, v1, k0, k1, v0, dma);
      if (kB) mma_phase(j, v1, k0, k1, v0, dma); else sm_phase(j);
      tile_barrier();
      if (j + 1 > j1) break;
      // tile j+1: K in k1, V in v1; tile j: V in v0; tile j+2: K in k0.
      if (kB) sm_phase(j); else mma_phase(j + 1, v0, k1, k0, v1, dma);
      if (kB) mma_phase(j + 1, v0, k1, k0, v1, dma); else sm_phase(j + 1);
      tile_barrier();
      if (j + 2 > j1) break;
    }
  };
  if (grp_b)
    run(BoolC<true>{});
  else
    run(BoolC<false>{});

  // Every wave is past the loop's last barrier: LDS and qf are free.
  const float l_all = half_sum(l_run);
  if constexpr (kEarlyOut) {
    if (row_valid) fwd_store_ptrs<T, Prob::kF32Out>(out_row, lse_row, lh, o, l_all, ms_run);
  } else {
    if (row_valid) fwd_store_row<T>(P, row, lh, o, l_all, ms_run);
  }
  if (!next(P, row0)) break;
  start_tile();
  }
}

// One row tile.
template <class T, class Prob>
__device__ __forceinline__ void attn_fwd_tile_d128(const Prob& P, int row0, float scale,
                                                   char* k0, char* v0, char* k1, char* v1) {
  attn_fwd_tiles_d128<T>(P, row0, scale, k0, v0, k1, v1, [](Prob&, int&) { return false; });
}

}  // namespace fa

