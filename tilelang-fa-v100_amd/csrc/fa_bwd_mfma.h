// Attention backward main kernel for head_dim 128 and 256 on gfx950.
//
// Same mathematics as bwd_main_kernel (fa_bwd.hip): per (key tile, query
// tile) the products S = Q Kᵀ, dP = dO Vᵀ, dVᵀ += dOᵀ P, dKᵀ += Qᵀ dS and,
// on the atomic path (DQ = true, head_dim 256 only), dQ += dS K, with
// P = exp2(S·scale·log2e − LSE·log2e) and dS = P (dP − rowdot).
// Layout, for the gfx950 memory instructions:
//  * D = 128 (dK / dV only; dQ from bwd_dq_kernel): 256 keys per
//    workgroup, NW = 8 / KB waves, each owning KB blocks of 32 keys, so every
//    Q / dO tile fetched into LDS serves 256 keys.  With KB = 2 (4 waves, one
//    per SIMD) a wave has 512 registers, holds dK / dV of 64 keys, and every
//    Q / dO operand it reads from LDS feeds the products of both its key
//    blocks.
//  * D = 256: 128 keys per workgroup, 4 waves x 32 keys, one wave per SIMD
//    (dK / dV of 32 keys x 256 d take 256 registers); rows are 512 bytes,
//    and on the atomic path each wave computes two 32-wide d tiles of dQ,
//    which the fp32 atomics then reduce across key tiles.
//  * The workgroup's K tile (BKV x 2D bytes) is copied once HBM -> LDS with
//    global_load_lds_dwordx4 and serves as the B operand of S (row reads)
//    and of dQ (transpose reads).  V rows of each wave stay in registers.
//  * Q and dO tiles (32 rows) are DMA'd through buffer resources
//    (buffer_load_dwordx4 ... lds), double-buffered in distinct arrays (see
//    attn_fwd_tile_d128 for why distinct arrays).  Qᵀ / dOᵀ operands come
//    from ds_read_b64_tr_b16; nothing is transposed in registers.
//  * dSᵀ goes to LDS (double-buffered) with 8-byte stores (its 8-byte
//    pieces XOR-swizzled by row so both the stores and the transpose reads
//    are conflict free) and is read back transposed as the A operand of dQ.
//    Four waves each compute the 32 x 32 dQ blocks of their d tiles over
//    all keys of the workgroup, one iteration later (after the single
//    barrier of the next iteration), so the dQ products overlap the S / dP
//    products of the next tile, and add it to the fp32 accumulator with
//    buffer atomics.
//  * K / Q / dO rows use the 16-byte-chunk swizzle of fa_fwd_d128.h on the
//    low four chunk bits (within each 256-byte half of a 512-byte row).
#pragma once

#include "fa355.h"
#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

template <int D_, int KB>
struct BwdShapeMfma {
  static constexpr int D = D_;
  static constexpr int NW = D == 128 ? 8 / KB : 4;  // waves per workgroup
  static constexpr int BKV = 32 * KB * NW;  // keys per workgroup: 256 (D=128), 128 (D=256)
  static constexpr int BQ = tiles::kBwdQueryRows;  // query rows per iteration
  static constexpr int ROWB = 2 * D;        // bytes per K / Q / dO row
  static constexpr int CPR = D / 8;         // 16-byte chunks per row
  static constexpr int RPB = 1024 / ROWB;   // rows per 1 KB DMA block
  static constexpr int K_BYTES = BKV * ROWB;  // 64 KB
  static constexpr int QT_BYTES = BQ * ROWB;  // 8 or 16 KB
  static constexpr int QT_BLOCKS = QT_BYTES / 1024;
  static constexpr int DS_ROWB = BQ * 2;      // 64 B per dSᵀ row
  static constexpr int DS_BYTES = BKV * DS_ROWB;  // double-buffered
  static constexpr int DQT = D / 32;          // 32-wide d tiles of dQ
  static constexpr int DQW = NW < DQT ? NW : DQT;  // waves computing dQ
  static constexpr int DTW = DQT / DQW;       // d tiles per dQ wave
  static constexpr int WPE = NW / 4;          // waves per SIMD
  static_assert(D == 128 || D == 256, "head_dim");
  static_assert(KB == 1 || (KB == 2 && D == 128), "key blocks per wave");
  static_assert(QT_BLOCKS % NW == 0 && (K_BYTES / 1024) % NW == 0, "DMA split");
};

// Key blocks per wave used by the launcher.
constexpr int kBwdKB = tiles::kBwd128KeyBlocksPerWave;

// MODE (MaskMode): full attention, causal, or a window band from the arguments.
// DQ: also compute dQ (dSᵀ through LDS, fp32 atomics into dqacc); without it
// the kernel writes dK / dV only and dQ comes from bwd_dq_kernel
// (fa_bwd_dq.h, the deterministic path).
template <class T, int D_, int MODE, int KB, bool DQ>
__global__ __launch_bounds__((64 * BwdShapeMfma<D_, KB>::NW), (BwdShapeMfma<D_, KB>::WPE))
void bwd_main_mfma_kernel(fa_bwd_args a, float* dqacc, const float* stats) {
  using S = BwdShapeMfma<D_, KB>;
  constexpr bool CAUSAL = MODE != kMaskNone;  // some (query, key) pairs are outside the band
  constexpr int D = S::D;
  // One LDS array.  The statistics and the Q / dO tiles come first, so
  // their array offsets are instruction immediates (the 16-bit offset field
  // reaches 64 KB); dSᵀ and K are addressed through per-lane bases that
  // include their offsets.  Bases are combined with XOR constants below bit
  // 9, so those offsets are multiples of 512.
  constexpr int OFF_ST0 = 0, OFF_ST1 = 2 * S::BQ * 4;
  constexpr int OFF_Q0 = 512, OFF_O0 = OFF_Q0 + S::QT_BYTES, OFF_Q1 = OFF_O0 + S::QT_BYTES,
                OFF_O1 = OFF_Q1 + S::QT_BYTES;
  constexpr int OFF_DS0 = OFF_O1 + S::QT_BYTES, OFF_DS1 = OFF_DS0 + S::DS_BYTES;
  constexpr int OFF_K = OFF_DS1 + S::DS_BYTES;
  static_assert(OFF_ST1 + 2 * S::BQ * 4 <= OFF_Q0 && OFF_K % 512 == 0 && OFF_DS0 % 512 == 0,
                "LDS layout");
  __shared__ __attribute__((aligned(16))) char smem[OFF_K + S::K_BYTES];
  char* const Ks = smem + OFF_K;

  const int Sq = a.seqlen_q, Sk = a.seqlen_k, H = a.num_heads, Hk = a.num_heads_k;
  const int G = H / Hk;
  const int kvtiles = (Sk + S::BKV - 1) / S::BKV;
  // Rank 0 = key tile 0, which sees the most query rows when causal.
  const TileHead th = xcd_tile_order(blockIdx.x, kvtiles, a.batch * Hk);
  const int kt_idx = th.rank;
  const int bh = th.bh;
  const int hk = bh % Hk, b = bh / Hk;
  const int kv0 = kt_idx * S::BKV;
  // Visible pairs: the band of MODE; with kMaskNone every (query, key) pair
  // inside the bounds.
  const Band band = mode_band<MODE>(a);
  const int off = band.off;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  // Key block kb of this wave: keys kvb(kb) .. kvb(kb) + 31; lane key kvb + lr.
  const int wrow = 32 * KB * wave;  // first key row of the wave within the tile
  auto kvb = [&](int kb) { return kv0 + wrow + 32 * kb; };
  const float scale_log2 = a.softmax_scale * kLog2e;

  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[2];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[2];

  // ---- K tile -> LDS: 64 blocks of 1 KB (RPB rows each); wave w loads the
  // blocks of its own key rows.
  constexpr int KBPW = S::K_BYTES / 1024 / S::NW;
#pragma unroll
  for (int ii = 0; ii < KBPW; ++ii) {
    const int blk = KBPW * wave + ii;
    const int r = S::RPB * blk + lane / S::CPR;
    const int c = (lane % S::CPR) ^ swz_chunk(r);
    const int n = min(kv0 + r, Sk - 1);
    load_lds16(kg + (int64_t)n * a.k_stride[1] + 8 * c, Ks + blk * 1024);
  }
  // ---- V rows of this wave (B operand of dP = dO Vᵀ)
  u32x4 vB[KB][D / 16];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const uint16_t* vp = vg + (int64_t)min(kvb(kb) + lr, Sk - 1) * a.v_stride[1];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) vB[kb][c] = ld16(vp + 16 * c + 8 * lh);
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
  // dSᵀ row wrow + 32kb + lr, piece 2g + lh: 8((2g + lh) ^ m) with
  // m = (row >> 2) & 7 = (lr >> 2) & 7 = 16(g ^ (m >> 1)) + 8(lh ^ (m & 1)).
  const int dsw_m = (lr >> 2) & 7;
  int dw = OFF_DS0 + (wrow + lr) * S::DS_ROWB + 16 * (dsw_m >> 1) + 8 * (lh ^ (dsw_m & 1));
  auto dsw_off = [&](int kb, int g) { return (dw ^ (16 * g)) + 32 * kb * S::DS_ROWB; };
  // dSᵀ transpose reads: rows 16kc + r (+8 for hf = 1), piece p =
  // 4((k/16)%2) + k%4 stored at p ^ m, m = (row >> 2) & 7 = (r >> 2) +
  // 4(kc & 1) + 2hf; all three terms occupy distinct bits, so the offset is
  // a base XOR 32(kc & 1) XOR 16hf, plus (16kc + 8hf) rows as an immediate.
  const int ds_r = 4 * (lane >> 5) + ((lane & 15) >> 2);
  const int ds_p = 4 * ((lane >> 4) & 1) + (lane & 3);
  int dsr = OFF_DS0 + ds_r * S::DS_ROWB + 8 * (ds_p ^ (ds_r >> 2));
  auto dsr_off = [&](int kc, int hf) {
    return (dsr ^ (32 * (kc & 1)) ^ (16 * hf)) + (16 * kc + 8 * hf) * S::DS_ROWB;
  };

  f32x16 dk[KB][D / 32], dv[KB][D / 32];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) dk[kb][dt][i] = dv[kb][dt][i] = 0.f;

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
  // from the tile's first row is fixed.  (Leaving the DMA to the waves
  // without dQ work, so that the dQ waves never wait for their atomics at
  // the barrier, measured slower.)
  constexpr int BPW = S::QT_BLOCKS / S::NW;
  uint32_t q_loff[BPW], o_loff[BPW];
#pragma unroll
  for (int ii = 0; ii < BPW; ++ii) {
    const int r = S::RPB * (BPW * wave + ii) + lane / S::CPR;
    const uint32_t c = (lane % S::CPR) ^ swz_chunk(r);
    q_loff[ii] = 2u * (r * (uint32_t)a.q_stride[1] + 8 * c);
    o_loff[ii] = 2u * (r * (uint32_t)a.do_stride[1] + 8 * c);
  }

  // Tile t covers query head hk*G + t / nit and query tile it1 - 1 - t % nit;
  // (h_rel, it) is carried incrementally so the loop has no integer division.
  auto issue_q = [&](int h_rel, int it, int qo, int oo, int so) {
    const int h = hk * G + h_rel;
    const int i0 = it * S::BQ;
    // Buffer resources over the tile's valid rows: rows at or past Sq read
    // as zero (their products are masked), so no row clamping is needed.
    const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + b * a.q_stride[0] +
                           h * a.q_stride[2] + (int64_t)i0 * a.q_stride[1];
    const uint16_t* orow = static_cast<const uint16_t*>(a.dout) + b * a.do_stride[0] +
                           h * a.do_stride[2] + (int64_t)i0 * a.do_stride[1];
    const uint32_t nrows = (uint32_t)min(Sq - i0, S::BQ);
    const u32x4 rq = rsrc_words(qrow, span_bytes(nrows, a.q_stride[1], D));
    const u32x4 ro = rsrc_words(orow, span_bytes(nrows, a.do_stride[1], D));
    // Opaque DMA: the loop's wait_vmem + barrier is the only wait the tile
    // needs (the compiler would otherwise wait for it, and for the dQ
    // atomics, before each dSᵀ access).
#pragma unroll
    for (int ii = 0; ii < BPW; ++ii) {
      const int blk = BPW * wave + ii;
      buffer_lds16_opaque(rq, q_loff[ii], smem + qo + blk * 1024);
      buffer_lds16_opaque(ro, o_loff[ii], smem + oo + blk * 1024);
    }
    if (wave == 0) {
      // Lanes 0-31 fetch LSE*log2(e), lanes 32-63 rowdot ([B*H][2][Sq]).
      const float* sbase = stats + 2 * (head_rows + h_rel) * Sq + i0;
      const unsigned lo = (lane >> 5) * Sq + min(lane & 31, Sq - 1 - i0);
      global_lds4_opaque(sbase + lo, smem + so);
    }
  };

  // S, dP, softmax, dSᵀ -> dsb, dV and dK for one query tile (no barrier).
  // qo, oo, so: offsets of the Q, dO and statistics tiles; dso: 0 for dSᵀ
  // buffer 0, DS_BYTES for buffer 1.
  auto step = [&](int h_rel, int it, int qo, int oo, int so, int dso) {
    const char* qb = smem + qo;
    const char* ob = smem + oo;
    const float* st = reinterpret_cast<const float*>(smem + so);
    // The per-chunk offsets are `base ^ constant`.  Marking the bases as
    // (opaquely) rewritten each iteration keeps the compiler from hoisting
    // every XOR result out of the loop into a register of its own.
    asm volatile("" : "+v"(rb), "+v"(tb0), "+v"(tb1), "+v"(dw), "+v"(rbk));
    const int i0 = it * S::BQ;
    // Key block 0 has the smallest keys: if it lies past Sk, no block of the
    // wave has keys.  Causal: the wave skips tiles none of its keys see.  A
    // general band runs such tiles through the masked path instead (P = 0):
    // its two-sided test makes the register allocator spill heavily, and
    // they are at most BKV / BQ tiles per workgroup.
    const bool active =
        (MODE != kMaskCausal || band.any(i0, i0 + S::BQ - 1, kvb(0), kvb(KB - 1) + 31)) &&
        kvb(0) < Sk;
    if (active) {
      f32x16 s[KB], dp[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[kb][i] = dp[kb][i] = 0.f;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const u32x4 aq = ld16(qb + rm_off(c));
        const u32x4 ao = ld16(ob + rm_off(c));
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const u32x4 bk = ld16(smem + rk_off(c) + 32 * kb * S::ROWB);
          s[kb] = T::mma32(aq, bk, s[kb]);
          dp[kb] = T::mma32(ao, vB[kb][c], dp[kb]);
        }
      }
      // Keep two chunks of operands in flight: loads of chunk c + 2 are
      // issued between the products of chunk c (bounds register use).
      sched_pipeline<D / 16, 2 + KB, 2 * KB, 2>();

      u32x4 pB[KB][2], sB[KB][2];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int kvw = kvb(kb);
        const int wkv_last = min(kvw + 31, Sk - 1);
        const bool need_mask = (CAUSAL && !band.all(i0, i0 + S::BQ - 1, kvw, wkv_last)) ||
                               (kvw + 32 > Sk) || (i0 + S::BQ > Sq);
        // P = exp2(S·scale·log2e − lse2), dS = P (dP − rowdot).  Element
        // (g, r) is query i0 + 8g + 4lh + r; on masked tiles it sees the
        // lane's key iff c = 8g + r lies in [t_lo, t_hi); masked elements
        // get P = 0.  The masked and unmasked forms are separate code paths
        // so that the uniform branch between them stays a branch.
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
              float p = fast_exp2(fmaf(s[kb][i], scale_log2, -l4[r]));
              if constexpr (kMasked) {
                const int c = 8 * g + r;
                p = (c >= t_lo && c < t_hi) ? p : 0.f;
              }
              s[kb][i] = p;
              dp[kb][i] = p * (dp[kb][i] - d4[r]);
            }
          }
        };
        if (need_mask)
          softmax(BoolC<true>{});
        else
          softmax(BoolC<false>{});
#pragma unroll
        for (int kq = 0; kq < 2; ++kq)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int e = 8 * kq + 2 * w;
            pB[kb][kq][w] = T::pack(s[kb][e], s[kb][e + 1]);
            sB[kb][kq][w] = T::pack(dp[kb][e], dp[kb][e + 1]);
          }
        // dSᵀ row wrow + 32kb + lr; queries 8g + 4lh .. +3 = piece 2g + lh.
        if constexpr (DQ) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int kq = g >> 1, w0 = 2 * (g & 1);
            const u32x2 v = {sB[kb][kq][w0], sB[kb][kq][w0 + 1]};
            st8(smem + dso + dsw_off(kb, g), v);
          }
        }
      }
      // dVᵀ += dOᵀ P, dKᵀ += Qᵀ dS   (A operands by transpose reads, shared
      // by the wave's key blocks)
#pragma unroll
      for (int kq = 0; kq < 2; ++kq)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const int ro = kq * 16 * S::ROWB;
          const u32x2 o_lo = lds_read_tr(ob + toff(0, dt) + ro);
          const u32x2 o_hi = lds_read_tr(ob + toff(1, dt) + ro);
          const u32x2 q_lo = lds_read_tr(qb + toff(0, dt) + ro);
          const u32x2 q_hi = lds_read_tr(qb + toff(1, dt) + ro);
          const u32x4 ao = {o_lo[0], o_lo[1], o_hi[0], o_hi[1]};
          const u32x4 aq = {q_lo[0], q_lo[1], q_hi[0], q_hi[1]};
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            dv[kb][dt] = T::mma32(ao, pB[kb][kq], dv[kb][dt]);
            dk[kb][dt] = T::mma32(aq, sB[kb][kq], dk[kb][dt]);
          }
        }
      sched_pipeline<2 * (D / 32), 4, 2 * KB, 2>();
    } else if constexpr (DQ) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) st8(smem + dso + dsw_off(kb, g), u32x2{0, 0});
    }
  };

  // dQ[i0 + q][32 dt + d] += sum over the workgroup's keys of dS K, for the
  // tile whose dSᵀ is complete in dsb (waves 0 .. DQW-1, d tiles
  // dt = wave + DQW j).
  auto dq_step = [&](int h_rel, int it, int dso) {
    if constexpr (!DQ) return;
    const int i0 = it * S::BQ;
    const bool any = !CAUSAL || band.any(i0, i0 + S::BQ - 1, kv0, kv0 + S::BKV - 1);
    if (wave < S::DQW && any) {
      asm volatile("" : "+v"(dsr));
      f32x16 acc[S::DTW];
#pragma unroll
      for (int j = 0; j < S::DTW; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.f;
      struct DqOps {
        u32x2 s_lo, s_hi, k_lo[S::DTW], k_hi[S::DTW];
      };
      lds_pipeline<S::BKV / 16, 2>(
          [&](int kc) {
            DqOps o;
            o.s_lo = lds_read_tr(smem + dso + dsr_off(kc, 0));
            o.s_hi = lds_read_tr(smem + dso + dsr_off(kc, 1));
            const int ro = kc * 16 * S::ROWB;
#pragma unroll
            for (int j = 0; j < S::DTW; ++j) {
              const int dt = wave + S::DQW * j;
              o.k_lo[j] = lds_read_tr(Ks + toff(0, dt) + ro);
              o.k_hi[j] = lds_read_tr(Ks + toff(1, dt) + ro);
            }
            return o;
          },
          [&](int, const DqOps& o) {
            const u32x4 as = {o.s_lo[0], o.s_lo[1], o.s_hi[0], o.s_hi[1]};
#pragma unroll
            for (int j = 0; j < S::DTW; ++j) {
              const u32x4 bk = {o.k_lo[j][0], o.k_lo[j][1], o.k_hi[j][0], o.k_hi[j][1]};
              acc[j] = T::mma32(as, bk, acc[j]);
            }
          });
      // acc[j][4g + r] = dQ[query i0 + 8g + 4lh + r][d 32dt + lr]; dqacc is
      // [B, H, Sq, D].  The resource ends after column 31 of the tile's last
      // valid row, so atomics for rows at or past Sq are dropped.
      const uint32_t nrows = (uint32_t)min(Sq - i0, S::BQ);
      const uint32_t lo = 4u * (4 * lh * D + lr);
#pragma unroll
      for (int j = 0; j < S::DTW; ++j) {
        const int dt = wave + S::DQW * j;
        const float* dqh = dqacc + ((head_rows + h_rel) * Sq + i0) * D + 32 * dt;
        const rsrc_t rd = make_rsrc(dqh, ((nrows - 1) * D + 32) * 4u);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            buffer_atomic_add(rd, lo, 4u * (8 * g + r) * D, acc[j][4 * g + r]);
      }
    }
  };

  // Query tiles are swept from the last down: the workgroups of one head
  // that run at the same time (consecutive key tiles) then add into the
  // same dQ rows at about the same time, which keeps those rows in L2 for
  // the atomics (measured ~3% faster than the ascending sweep).
  int ih = 0, ii = it1 - 1;  // tile to issue next
  int ch = 0, ci = it1 - 1;  // tile to compute next
  auto advance = [&](int& h_rel, int& it) {
    if (it-- == it0) {
      it = it1 - 1;
      ++h_rel;
    }
  };
  // Iteration t: one barrier (Q/dO tile t landed, dSᵀ of tile t-1 complete,
  // buffers of tile t-1 free), then the DMA of tile t+1, the dQ product of
  // tile t-1 (overlapping other waves' products of tile t) and tile t's
  // products.  dSᵀ alternates between dS0 and dS1.
  int ph = 0, pi = 0;  // tile whose dQ is pending
  if (ntot > 0) {
    issue_q(ih, ii, OFF_Q0, OFF_O0, OFF_ST0);
    advance(ih, ii);
  }
  for (int t = 0; t < ntot; t += 2) {
    wait_vmem();
    __syncthreads();
    if (t + 1 < ntot) {
      issue_q(ih, ii, OFF_Q1, OFF_O1, OFF_ST1);
      advance(ih, ii);
    }
    if (t > 0) dq_step(ph, pi, S::DS_BYTES);
    __builtin_amdgcn_sched_barrier(0);  // keep the two phases' registers apart
    step(ch, ci, OFF_Q0, OFF_O0, OFF_ST0, 0);
    ph = ch;
    pi = ci;
    advance(ch, ci);
    if (t + 1 < ntot) {
      wait_vmem();
      __syncthreads();
      if (t + 2 < ntot) {
        issue_q(ih, ii, OFF_Q0, OFF_O0, OFF_ST0);
        advance(ih, ii);
      }
      dq_step(ph, pi, 0);
      __builtin_amdgcn_sched_barrier(0);
      step(ch, ci, OFF_Q1, OFF_O1, OFF_ST1, S::DS_BYTES);
      ph = ch;
      pi = ci;
      advance(ch, ci);
    }
  }
  if (ntot > 0) {
    __syncthreads();  // dSᵀ of the last tile complete
    dq_step(ph, pi, ((ntot - 1) & 1) ? S::DS_BYTES : 0);
  }
  wait_vmem();

  const float sc = a.softmax_scale;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int my_kv = kvb(kb) + lr;
    if (my_kv >= Sk) continue;
    uint16_t* dkp = static_cast<uint16_t*>(a.dk) + b * a.dk_stride[0] +
                    (int64_t)my_kv * a.dk_stride[1] + hk * a.dk_stride[2];
    uint16_t* dvp = static_cast<uint16_t*>(a.dv) + b * a.dv_stride[0] +
                    (int64_t)my_kv * a.dv_stride[1] + hk * a.dv_stride[2];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * lh;
        u32x2 wk, wv;
        wk[0] = T::pack(dk[kb][dt][4 * g] * sc, dk[kb][dt][4 * g + 1] * sc);
        wk[1] = T::pack(dk[kb][dt][4 * g + 2] * sc, dk[kb][dt][4 * g + 3] * sc);
        wv[0] = T::pack(dv[kb][dt][4 * g], dv[kb][dt][4 * g + 1]);
        wv[1] = T::pack(dv[kb][dt][4 * g + 2], dv[kb][dt][4 * g + 3]);
        st8(dkp + d, wk);
        st8(dvp + d, wv);
      }
  }
}

}  // namespace fa
