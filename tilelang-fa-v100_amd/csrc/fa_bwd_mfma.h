// Key-stationary attention backward (dK, dV) for head_dim 128 and 256 on gfx950.
//
// Same mathematics as bwd_main_kernel (fa_bwd.hip): per (key tile, query
// tile) the products S = Q Kᵀ, dP = dO Vᵀ, dVᵀ += dOᵀ P and dKᵀ += Qᵀ dS, with
// P = exp2(S·scale·log2e − LSE·log2e) and dS = P (dP − rowdot)·scale (rounded
// to 16 bits with the scale in, as the reference does,
// tilelang_fa_v100/_kernels_backward.py:160); dQ comes from
// the query-stationary bwd_dq_kernel (fa_bwd_dq.h).  Layout, for the gfx950
// memory instructions:
//  * D = 128: 256 keys per workgroup, 8 waves x 32 keys (two waves per SIMD),
//    so every Q / dO tile fetched into LDS serves 256 keys.
//  * D = 256: 128 keys per workgroup, 4 waves x 32 keys, one wave per SIMD
//    (dK / dV of 32 keys x 256 d take 256 registers); rows are 512 bytes.
//  * The workgroup's K tile (BKV x 2D bytes) is copied once HBM -> LDS with
//    global_load_lds_dwordx4 and serves as the B operand of S (row reads).
//    V rows of each wave stay in registers.
//  * Q and dO tiles (32 rows) are DMA'd through buffer resources
//    (buffer_load_dwordx4 ... lds), double-buffered.  Qᵀ / dOᵀ operands come
//    from ds_read_b64_tr_b16; nothing is transposed in registers.
//  * K / Q / dO rows use the 16-byte-chunk swizzle of fa_fwd_d128.h on the
//    low four chunk bits (within each 256-byte half of a 512-byte row).
#pragma once

#include "fa355.h"
#include "fa_bwd_ds.h"
#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

template <int D_>
struct BwdShapeMfma {
  static constexpr int D = D_;
  static constexpr int NW = D == 128 ? 8 : 4;  // waves per workgroup
  static constexpr int BKV = 32 * NW;       // keys per workgroup: 256 (D=128), 128 (D=256)
  static constexpr int BQ = tiles::kBwdQueryRows;  // query rows per iteration
  static constexpr int ROWB = 2 * D;        // bytes per K / Q / dO row
  static constexpr int CPR = D / 8;         // 16-byte chunks per row
  static constexpr int RPB = 1024 / ROWB;   // rows per 1 KB DMA block
  static constexpr int K_BYTES = BKV * ROWB;  // 64 KB
  static constexpr int QT_BYTES = BQ * ROWB;  // 8 or 16 KB
  static constexpr int QT_BLOCKS = QT_BYTES / 1024;
  static constexpr int WPE = NW / 4;          // waves per SIMD
  static_assert(D == 128 || D == 256, "head_dim");
  static_assert(QT_BLOCKS % NW == 0 && (K_BYTES / 1024) % NW == 0, "DMA split");
};

// A operands (dOᵀ, Qᵀ) of one dVᵀ / dKᵀ product pair.
struct TrOps {
  u32x4 ao, aq;
};

// MODE (MaskMode): full attention, causal, or a window band from the arguments.
// DS: also store every computed 32 x 32 dS block to `ds` (tile layout of
// fa_bwd_ds.h; causal or full attention) for bwd_dq_ds_kernel.
template <class T, int D_, int MODE, bool DS = false>
__global__ __launch_bounds__((64 * BwdShapeMfma<D_>::NW), (BwdShapeMfma<D_>::WPE))
void bwd_main_mfma_kernel(fa_bwd_args a, const float* stats, uint16_t* ds) {
  using S = BwdShapeMfma<D_>;
  constexpr bool CAUSAL = MODE != kMaskNone;  // some (query, key) pairs are outside the band
  constexpr int D = S::D;
  // One LDS array.  The statistics and the Q / dO tiles come first, so
  // their array offsets are instruction immediates (the 16-bit offset field
  // reaches 64 KB); K is addressed through a per-lane base that includes its
  // offset.  Bases are combined with XOR constants below bit 9, so that
  // offset is a multiple of 512.
  constexpr int OFF_ST0 = 0, OFF_ST1 = 2 * S::BQ * 4;
  constexpr int OFF_Q0 = 512, OFF_O0 = OFF_Q0 + S::QT_BYTES, OFF_Q1 = OFF_O0 + S::QT_BYTES,
                OFF_O1 = OFF_Q1 + S::QT_BYTES;
  constexpr int OFF_K = OFF_O1 + S::QT_BYTES;
  static_assert(OFF_ST1 + 2 * S::BQ * 4 <= OFF_Q0 && OFF_K % 512 == 0, "LDS layout");
  static_assert(OFF_O0 - OFF_Q0 == S::QT_BYTES && OFF_O1 - OFF_Q1 == S::QT_BYTES, "dO after Q");
  __shared__ __attribute__((aligned(16))) char smem[OFF_K + S::K_BYTES];
  char* const Ks = smem + OFF_K;

  const int Sq = a.seqlen_q, Sk = a.seqlen_k, H = a.num_heads, Hk = a.num_heads_k;
  const int G = H / Hk;
  const int kvtiles = (Sk + S::BKV - 1) / S::BKV;
  // Rank 0 = key tile 0, which sees the most query rows when causal.
  const TileHead th = xcd_tile_order(blockIdx.x, kvtiles, a.batch * Hk);
  const int bh = th.bh;
  const int hk = bh % Hk, b = bh / Hk;
  const int kv0 = th.rank * S::BKV;
  // Visible pairs: the band of MODE; with kMaskNone every (query, key) pair
  // inside the bounds.
  const Band band = mode_band<MODE>(a);
  const int off = band.off;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  // The wave's keys: kvw .. kvw + 31; lane key kvw + lr.
  const int wrow = 32 * wave;  // first key row of the wave within the tile
  const int kvw = kv0 + wrow;
  const float scale_log2 = a.softmax_scale * kLog2e;
  const float sc = a.softmax_scale;

  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[2];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[2];
  // This lane's dK / dV rows (key kvw + lr), formed here and held in VGPRs:
  // formed after the loop, their arguments (pointers and strides) stayed
  // live through it as one 16-register scalar tuple, which spilled and was
  // reloaded every iteration (16 v_readlane per tile; T1 backward 1.591 ->
  // 1.547 ms, head_dim 256 1.535 -> 1.486 ms without them, same box).
  uint16_t* dkp = static_cast<uint16_t*>(a.dk) + b * a.dk_stride[0] +
                  (int64_t)(kvw + lr) * a.dk_stride[1] + hk * a.dk_stride[2];
  uint16_t* dvp = static_cast<uint16_t*>(a.dv) + b * a.dv_stride[0] +
                  (int64_t)(kvw + lr) * a.dv_stride[1] + hk * a.dv_stride[2];
  asm volatile("" : "+v"(dkp), "+v"(dvp));

  // ---- K tile -> LDS: 1 KB blocks of RPB rows; wave w loads the blocks of
  // its own key rows.
  constexpr int KBPW = S::K_BYTES / 1024 / S::NW;
#pragma unroll
  for (int ii = 0; ii < KBPW; ++ii) {
    const int blk = KBPW * wave + ii;
    const int r = S::RPB * blk + lane / S::CPR;
    const int c = (lane % S::CPR) ^ swz_chunk(r);
    const int n = min(kv0 + r, Sk - 1);
    global_lds16_opaque(kg + (int64_t)n * a.k_stride[1] + 8 * c, Ks + blk * 1024);
  }
  // ---- V rows of this wave (B operand of dP = dO Vᵀ)
  u32x4 vB[D / 16];
  {
    const uint16_t* vp = vg + (int64_t)min(kvw + lr, Sk - 1) * a.v_stride[1];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) vB[c] = ld16(vp + 16 * c + 8 * lh);
  }

  // ---- per-lane LDS offsets.  Chunk c of row r sits at chunk c ^ swz(r);
  // the chunk-index bits a product walks (c for row reads, the 64-byte d
  // tile for transpose reads) are free in the lane's base offset, so every
  // offset is that base XOR an instruction constant (one register per
  // pattern instead of one per chunk).  Row offsets of 16-row multiples are
  // instruction immediates.
  const int sw_lr = swz_chunk(lr);
  // Row read of chunk pair c (row lr, chunk 2c + lh):
  // 16((2c + lh) ^ sw) = 32(c ^ (sw >> 1)) + 16(lh ^ (sw & 1)).
  int rb = lr * S::ROWB + 16 * (lh ^ (sw_lr & 1)) + 32 * (sw_lr >> 1);
  auto rm_off = [&](int c) { return rb ^ (32 * c); };
  // The same for the wave's own K rows (array offset included).
  int rbk = rb + OFF_K + wrow * S::ROWB;
  auto rk_off = [&](int c) { return rbk ^ (32 * c); };
  // Transpose read of rows 16k + r (r = 4(lane/32) + (lane%16)/4, +8 for
  // hf = 1), columns 32dt + 16((lane/16)%2) + 4(lane%4) of a 256 B-row tile:
  // 16((4dt + q) ^ swz(r)) = 64(dt ^ (r & 3)) + 16(q ^ ((r >> 2) & 3)).
  const int tr_r0 = 4 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_q = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  auto tr_base = [&](int hf) {
    const int r = tr_r0 + 8 * hf;
    return r * S::ROWB + 64 * (r & 3) + 16 * (tr_q ^ ((r >> 2) & 3)) + 8 * (lane & 1);
  };
  int tb0 = tr_base(0), tb1 = tr_base(1);
  auto toff = [&](int hf, int dt) { return (hf ? tb1 : tb0) ^ (64 * dt); };

  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) dk[dt][i] = dv[dt][i] = 0.f;
  // D = 256: dK / dV (32 keys x 256 d) fill the 256 AGPRs and stay there
  // (mma32_agpr); everything else fits the 256 VGPRs.
  if constexpr (D == 256) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      agpr_fence_in(dk[dt]);
      agpr_fence_in(dv[dt]);
    }
  }

  const int q_begin = CAUSAL ? band.first_row(kv0) : 0;
  const int q_end = CAUSAL ? band.end_row(kv0 + S::BKV - 1, Sq) : Sq;
  const int it0 = q_begin / S::BQ;
  const int it1 = (q_end + S::BQ - 1) / S::BQ;
  const int nit = max(it1 - it0, 0);
  const int ntot = nit * G;
  const int64_t head_rows = (int64_t)b * H + hk * G;  // (b, first query head) row block

  // Q / dO tile loader: 32 rows = QT_BLOCKS blocks of 1 KB; each wave loads
  // QT_BLOCKS / NW of them.  Lane l of block blk holds row RPB blk + l/CPR,
  // stored chunk l%CPR (logical chunk (l%CPR) ^ swz(row)); its byte offset
  // from the tile's first row is fixed.
  constexpr int BPW = S::QT_BLOCKS / S::NW;
  uint32_t q_loff[BPW], o_loff[BPW];
#pragma unroll
  for (int ii = 0; ii < BPW; ++ii) {
    const int r = S::RPB * (BPW * wave + ii) + lane / S::CPR;
    const uint32_t c = (lane % S::CPR) ^ swz_chunk(r);
    q_loff[ii] = 2u * (r * (uint32_t)a.q_stride[1] + 8 * c);
    o_loff[ii] = 2u * (r * (uint32_t)a.do_stride[1] + 8 * c);
  }

  // Tile t covers query head hk*G + t / nit and query tile it1 - 1 - t % nit
  // (query tiles are swept from the last down within each head).  The tile
  // to issue next is carried as (h_rel, it) and as running addresses of its
  // first Q / dO row and statistics, stepped back by one tile per iteration
  // and rebuilt when the head changes: no integer division and no 64-bit
  // products per tile (those were ~100 scalar instructions per tile).
  const int64_t qs1 = a.q_stride[1], os1 = a.do_stride[1];
  const uint16_t* q_top = static_cast<const uint16_t*>(a.q) + b * a.q_stride[0] +
                          (int64_t)(hk * G) * a.q_stride[2] + (int64_t)(max(it1, 1) - 1) * S::BQ * qs1;
  const uint16_t* o_top = static_cast<const uint16_t*>(a.dout) + b * a.do_stride[0] +
                          (int64_t)(hk * G) * a.do_stride[2] +
                          (int64_t)(max(it1, 1) - 1) * S::BQ * os1;
  const float* s_top = stats + 2 * head_rows * Sq + (max(it1, 1) - 1) * S::BQ;
  const float* s_i = s_top;
  // DS: the dS tile of the tile `step` computes next (same sweep order as
  // the issue side), stepped back by count(it) tiles per query tile.
  static_assert(!DS || MODE != kMaskBand, "dS tiles: causal or full attention");
  DsTiles dsl{1, 1, 1};
  uint16_t* ds_top = nullptr;
  if constexpr (DS) {
    dsl = ds_tiles<(MODE == kMaskCausal ? kMaskCausal : kMaskNone)>(Sq, Sk);
    ds_top = ds + 1024 * ((int64_t)(b * H + hk * G) * dsl.per_head() +
                          dsl.prefix(max(it1, 1) - 1) + kvw / 32);
  }
  uint16_t* ds_c = ds_top;
  // Buffer resources of the tile to issue next, based at its first Q / dO
  // row and carried from tile to tile: stepping back one tile is a 64-bit
  // subtract of the base words, and num_records (bytes up to the end of the
  // tile's last valid row) only differs on a head's first tile, the one that
  // may end at row Sq (rows at or past Sq read as zero; their products are
  // masked).  Built from the tile's row count every tile, the two resources
  // took ~25 scalar instructions per tile.
  const uint32_t q_full = span_bytes(S::BQ, qs1, D), o_full = span_bytes(S::BQ, os1, D);
  const int n_first = min(Sq - (max(it1, 1) - 1) * S::BQ, S::BQ);
  u32x4 rq = rsrc_words(q_top, span_bytes(n_first, qs1, D));
  u32x4 ro = rsrc_words(o_top, span_bytes(n_first, os1, D));
  auto step_back = [](u32x4& r, uint64_t bytes, uint32_t span) {
    const uint64_t p = (((uint64_t)r[1]) << 32 | r[0]) - bytes;
    r[0] = (uint32_t)p;
    r[1] = (uint32_t)(p >> 32);
    r[2] = span;
  };
  // Q / dO / statistics DMA of query tile `it` into the buffer at qo (the
  // dO tile sits QT_BYTES after the Q tile) and so.
  auto issue_q = [&](int it, int qo, int so) {
    const int i0 = it * S::BQ;
    // Opaque DMA: the loop's wait_vmem + barrier is the only wait the tile
    // needs.
#pragma unroll
    for (int ii = 0; ii < BPW; ++ii) {
      const int blk = BPW * wave + ii;
      buffer_lds16_pair<S::QT_BYTES>(rq, q_loff[ii], ro, o_loff[ii], smem + qo + blk * 1024);
    }
    if (wave == 0) {
      // Lanes 0-31 fetch LSE*log2(e), lanes 32-63 rowdot ([B*H][2][Sq]).
      const unsigned lo = (lane >> 5) * Sq + min(lane & 31, Sq - 1 - i0);
      global_lds4_opaque(s_i + lo, smem + so);
    }
  };
  // The next tile to issue, and its addresses.
  auto advance_issue = [&](int& h_rel, int& it) {
    if (it-- == it0) {
      it = it1 - 1;
      ++h_rel;
      s_i = s_top + 2 * h_rel * Sq;
      rq = rsrc_words(q_top + h_rel * a.q_stride[2], span_bytes(n_first, qs1, D));
      ro = rsrc_words(o_top + h_rel * a.do_stride[2], span_bytes(n_first, os1, D));
    } else {
      step_back(rq, 2ull * S::BQ * (uint64_t)qs1, q_full);
      step_back(ro, 2ull * S::BQ * (uint64_t)os1, o_full);
      s_i -= S::BQ;
    }
  };

  // S, dP, softmax, dV and dK for query tile `it` (no barrier).  qo, oo, so:
  // offsets of its Q, dO and statistics tiles.  Returns whether the wave
  // stored a dS tile (DS: two global stores, the wave's newest memory
  // operations).
  // Causal / full attention: tile `it` (rows i0 .. i0 + BQ - 1) is active
  // for this wave iff i0 >= act_lo (some row sees key kvw: kvw <= i0 + BQ - 1
  // + off) and needs no mask iff unm_lo <= i0 <= unm_hi (every row sees the
  // wave's last key, the wave's 32 keys and the tile's rows all exist): two
  // comparisons per tile instead of the band tests.
  const int wkv_last = min(kvw + 31, Sk - 1);
  constexpr int kNever = 0x7fffffff, kAlways = -0x7fffffff;
  const int act_lo = kvw >= Sk ? kNever : MODE == kMaskCausal ? kvw - (S::BQ - 1) - off : kAlways;
  const int unm_lo = kvw + 32 > Sk ? kNever : MODE == kMaskCausal ? wkv_last - off : kAlways;
  const int unm_hi = Sq - S::BQ;
  auto step = [&](int it, int qo, int oo, int so) -> bool {
    const char* qb = smem + qo;
    const char* ob = smem + oo;
    const float* st = reinterpret_cast<const float*>(smem + so);
    // The per-chunk offsets are `base ^ constant`.  Marking the bases as
    // (opaquely) rewritten each iteration keeps the compiler from hoisting
    // every XOR result out of the loop into a register of its own.
    asm volatile("" : "+v"(rb), "+v"(tb0), "+v"(tb1), "+v"(rbk));
    const int i0 = it * S::BQ;
    // Causal: the wave skips tiles none of its keys see.  A general band
    // runs such tiles through the masked path instead (P = 0): its two-sided
    // test makes the register allocator spill heavily, and they are at most
    // BKV / BQ tiles per workgroup.
    const bool active = MODE == kMaskBand ? kvw < Sk : i0 >= act_lo;
    if (!active) return false;
    f32x16 s, dp;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = dp[i] = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const u32x4 aq = ld16(qb + rm_off(c));
      const u32x4 ao = ld16(ob + rm_off(c));
      const u32x4 bk = ld16(smem + rk_off(c));
      s = T::mma32(aq, bk, s);
      dp = T::mma32(ao, vB[c], dp);
    }
    // Keep two chunks of operands in flight: loads of chunk c + 2 are
    // issued between the products of chunk c (bounds register use).
    sched_pipeline<D / 16, 3, 2, 2>();

    const bool need_mask =
        MODE == kMaskBand
            ? !band.all(i0, i0 + S::BQ - 1, kvw, wkv_last) || (kvw + 32 > Sk) || (i0 + S::BQ > Sq)
            : i0 < unm_lo || i0 > unm_hi;
    // P = exp2(S·scale·log2e − lse2), dS = P (dP·scale − scale·rowdot).  The
    // statistics hold scale·rowdot, so the scale costs nothing.  Element (g, r)
    // is query i0 + 8g + 4lh + r; on masked tiles it sees the lane's key iff
    // c = 8g + r lies in [t_lo, t_hi); masked elements get P = 0.  The
    // masked and unmasked forms are separate code paths so that the uniform
    // branch between them stays a branch.
    auto softmax = [&](auto masked) {
      constexpr bool kMasked = decltype(masked)::value;
      const int rel = i0 + 4 * lh;
      const int my_kv = kvw + lr;
      // j <= i + off + wr  <=>  c >= j - off - wr - rel;
      // j >= i + off - wl  <=>  c <= j - off + wl - rel.
      const int t_lo = (CAUSAL && band.wr >= 0) ? my_kv - off - band.wr - rel : -0x40000000;
      int t_hi = (my_kv < Sk) ? Sq - rel : -0x40000000;
      if (CAUSAL && band.wl >= 0) t_hi = min(t_hi, my_kv - off + band.wl - rel + 1);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int qb4 = 8 * g + 4 * lh;
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(st + qb4);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(st + S::BQ + qb4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 4 * g + r;
          float p = fast_exp2(fmaf(s[i], scale_log2, -l4[r]));
          if constexpr (kMasked) {
            const int c = 8 * g + r;
            p = (c >= t_lo && c < t_hi) ? p : 0.f;
          }
          s[i] = p;
          dp[i] = p * fmaf(dp[i], sc, -d4[r]);
        }
      }
    };
    if (need_mask)
      softmax(BoolC<true>{});
    else
      softmax(BoolC<false>{});
    u32x4 pB[2], sB[2];
#pragma unroll
    for (int kq = 0; kq < 2; ++kq)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e = 8 * kq + 2 * w;
        pB[kq][w] = T::pack(s[e], s[e + 1]);
        sB[kq][w] = T::pack(dp[e], dp[e + 1]);
      }
    if constexpr (DS) {
      // Chunk kq of lane (lr, lh) goes to 16-byte row 16(2(lr/16) + (lr/8)%2)
      // + 8lh + 4(((lr/4)%2) ^ kq) + lr%4 of the tile's 1 KB block kq, so
      // each store writes one whole block (layout in fa_bwd_ds.h).
      const int prow = 16 * (2 * (lr >> 4) + ((lr >> 3) & 1)) + 8 * lh + (lr & 3);
      const int g1 = (lr >> 2) & 1;
      ds_store16(ds_c + 8 * (prow + 4 * g1), sB[0]);
      ds_store16(ds_c + 512 + 8 * (prow + 4 * (g1 ^ 1)), sB[1]);
    }
    // dVᵀ += dOᵀ P, dKᵀ += Qᵀ dS   (A operands by transpose reads)
    auto tr_ops = [&](int kq, int dt) {
      const int ro = kq * 16 * S::ROWB;
      const u32x2 o_lo = lds_read_tr(ob + toff(0, dt) + ro);
      const u32x2 o_hi = lds_read_tr(ob + toff(1, dt) + ro);
      const u32x2 q_lo = lds_read_tr(qb + toff(0, dt) + ro);
      const u32x2 q_hi = lds_read_tr(qb + toff(1, dt) + ro);
      return TrOps{{o_lo[0], o_lo[1], o_hi[0], o_hi[1]}, {q_lo[0], q_lo[1], q_hi[0], q_hi[1]}};
    };
    if constexpr (D == 256) {
      lds_pipeline<2 * (D / 32), 2>(
          [&](int k) { return tr_ops(k / (D / 32), k % (D / 32)); },
          [&](int k, const TrOps& o) {
            const int kq = k / (D / 32), dt = k % (D / 32);
            mma32_agpr<T>(dv[dt], o.ao, pB[kq]);
            mma32_agpr<T>(dk[dt], o.aq, sB[kq]);
          });
    } else {
#pragma unroll
      for (int kq = 0; kq < 2; ++kq)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const TrOps o = tr_ops(kq, dt);
          dv[dt] = T::mma32(o.ao, pB[kq], dv[dt]);
          dk[dt] = T::mma32(o.aq, sB[kq], dk[dt]);
        }
      sched_pipeline<2 * (D / 32), 4, 2, 2>();
    }
    return DS;
  };

  auto advance = [&](int& h_rel, int& it) {
    if (it-- == it0) {
      it = it1 - 1;
      ++h_rel;
      if constexpr (DS) ds_c = ds_top + 1024 * h_rel * dsl.per_head();
    } else if constexpr (DS) {
      ds_c -= 1024 * dsl.count(it);
    }
  };
  int ih = 0, ii = it1 - 1;  // tile to issue next
  int ch = 0, ci = it1 - 1;  // tile to compute next
  // Iteration t: one barrier (Q/dO tile t landed, buffers of tile t-1 free),
  // then the DMA of tile t+1 and tile t's products.  The loop covers two
  // tiles so that every buffer offset is an instruction immediate.  The
  // wait before the barrier covers this wave's DMAs; the dS stores of the
  // step before, issued after them, stay in flight (vector memory counts
  // retire in issue order).
  auto wait_tile = [&](bool stored) {
    if (DS && stored)
      __builtin_amdgcn_s_waitcnt(0x0F72);
    else
      wait_vmem();
  };
  bool stored = false;
  if (ntot > 0) {
    issue_q(ii, OFF_Q0, OFF_ST0);
    advance_issue(ih, ii);
  }
  for (int t = 0; t < ntot; t += 2) {
    wait_tile(stored);
    __syncthreads();
    if (t + 1 < ntot) {
      issue_q(ii, OFF_Q1, OFF_ST1);
      advance_issue(ih, ii);
    }
    stored = step(ci, OFF_Q0, OFF_O0, OFF_ST0);
    advance(ch, ci);
    if (t + 1 >= ntot) break;
    wait_tile(stored);
    __syncthreads();
    if (t + 2 < ntot) {
      issue_q(ii, OFF_Q0, OFF_ST0);
      advance_issue(ih, ii);
    }
    stored = step(ci, OFF_Q1, OFF_O1, OFF_ST1);
    advance(ch, ci);
  }
  wait_vmem();
  if constexpr (D == 256) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      agpr_fence_out(dk[dt]);
      agpr_fence_out(dv[dt]);
    }
  }

  if (kvw + lr >= Sk) return;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
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

}  // namespace fa
