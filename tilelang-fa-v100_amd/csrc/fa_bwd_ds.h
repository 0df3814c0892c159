// dQ of the dense attention backward from stored dS tiles (head_dim 128 and
// 256, causal or full attention).
//
// The key-stationary dK / dV kernel (fa_bwd_mfma.h) forms dS = P (dP −
// rowdot)·scale for every (query tile, key block) pair it visits.  With its
// DS variant it also stores each wave's 32 x 32 block of dS (the 16-bit B
// operand of its dKᵀ product, 2 KB) to the workspace, and dQ = dS K becomes
// one product per tile pair (bwd_dq_ds_kernel) instead of the three of
// bwd_dq_kernel (fa_bwd_dq.h), which recomputes S and dP.  The price is
// writing and reading dS once through HBM (2 bytes per visible (query, key)
// pair).  Every dQ element is still summed by one lane over the keys in a
// fixed order, so the results repeat bit for bit, like the reference's
// query-stationary dQ kernel (tilelang_fa_v100/_kernels_backward.py:10-85).
//
// Tile layout: query head bh = b·H + h, query tile qt (rows 32qt..32qt+31)
// and key block kb (keys 32kb..32kb+31) with kb < count(qt) own the 2 KB at
//   ds + 2048 · (bh · per_head + prefix(qt) + kb),
// prefix(qt) = Σ_{t<qt} count(t).  A tile is two 1 KB blocks kq = 0, 1; lane
// (key, half) of the writing wave packs dS of query rows 16kq + 8(x/4) +
// 4 half + x%4, x = 0..7, as its chunk kq and stores it as 16-byte row
// 16(2(key/16) + (key/8)%2) + 8 half + 4(((key/4)%2) ^ kq) + key%4 of block kq:
// every store instruction writes one whole block, and the transposed reads
// of bwd_dq_ds_kernel hit 32 distinct 8-byte bank groups per half wave.

#pragma once

#include "fa355.h"
#include "fa_common.h"
#include "fa_fwd_d128.h"

namespace fa {

// dS tiles are written once and read once: both sides use the non-temporal
// (streaming) cache policy (measured at T1: dQ kernel 519 -> 467 us, the
// dK / dV kernel unchanged).
__device__ __forceinline__ void ds_store16(uint16_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// buffer_lds16_opaque with the non-temporal cache policy, twice: bytes voff
// and voff + 1024 of the resource into lds_block and lds_block + 1024, under
// one M0 value (the instruction offset applies to the memory address and to
// the LDS address alike).
__device__ __forceinline__ void buffer_lds16_stream2(u32x4 rsrc, uint32_t voff, char* lds_block) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen nt lds\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen offset:1024 nt lds\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(lds_addr(lds_block))
      : "memory");
}

// Per-head tile counts of the dS workspace.  count(t): key blocks a query
// tile reaches; causal (keys j <= i + Sk - Sq): kb <= t + floor((31 + Sk -
// Sq) / 32), clipped to [0, nk]; full attention: every block.
struct DsTiles {
  int nq, nk, c1;
  __host__ __device__ int count(int t) const { return min(max(t + c1, 0), nk); }
  // Σ_{t<n} count(t): zero below t0 = -c1, t + c1 up to t = nk - c1, then nk.
  __host__ __device__ int64_t prefix(int n) const {
    const int t0 = max(0, -c1);
    if (n <= t0) return 0;
    const int t1 = min(n, max(t0, nk - c1 + 1));
    const int64_t ramp = (int64_t)(t1 - t0) * (t0 + t1 - 1 + 2 * c1) / 2;
    return ramp + (int64_t)(n - t1) * nk;
  }
  __host__ __device__ int64_t per_head() const { return prefix(nq); }
};

__host__ __device__ inline int floor_div32(int x) { return x >= 0 ? x / 32 : -((31 - x) / 32); }

template <int MODE>
__host__ __device__ inline DsTiles ds_tiles(int sq, int sk) {
  static_assert(MODE == kMaskCausal || MODE == kMaskNone, "dS tiles: causal or full");
  const int nq = (sq + 31) / 32, nk = (sk + 31) / 32;
  const int c1 = MODE == kMaskCausal ? floor_div32(31 + sk - sq) + 1 : nk;
  return DsTiles{nq, nk, c1};
}

// Row statistics [B*H][2][Sq] fp32 for the dK / dV kernel: LSE·log2(e) (+inf
// for a row that saw no key, so that P is exactly zero) and scale·rowdot,
// rowdot = Σ_d O·dO (the reference's row_dot, _kernels_backward.py:203), with
// the arithmetic
// bwd_dq_kernel uses when it writes them: lanes l and l + 32 each sum half of
// every 16-column chunk with v_dot2, then the two halves are added.  Each wave
// takes kStatsTiles consecutive 32-row blocks of the (batch·head, row block)
// space and issues all their loads before the first sum (one wave per block
// took C2 15.6 / T1 35.2 us against 12.8 / 30.4 with four).
template <int D>
struct StatsShape {
  static constexpr int kTiles = D <= 128 ? 4 : 2;  // 250 / 198 VGPRs
};
template <class T, int D>
__global__ __launch_bounds__(256) void bwd_stats_kernel(fa_bwd_args a, float* stats) {
  constexpr int TPW = StatsShape<D>::kTiles;
  const int Sq = a.seqlen_q, H = a.num_heads;
  const int tiles = (Sq + 31) / 32;
  const int ntot = a.batch * H * tiles;
  const int gw0 = (blockIdx.x * 4 + wave_id()) * TPW;
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  u32x4 df[TPW][D / 16], ov[TPW][D / 16];
  float l[TPW];
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    // Blocks past the last repeat it (loaded, not stored).
    const int gw = min(gw0 + k, ntot - 1);
    const int bh = gw / tiles;
    const int row = (gw % tiles) * 32 + lr;
    const int h = bh % H, b = bh / H;
    const int64_t r = min(row, Sq - 1);
    // Issued first: its latency overlaps the row loads below.
    l[k] = a.lse[(int64_t)bh * Sq + r];
    const uint16_t* dp = static_cast<const uint16_t*>(a.dout) + b * a.do_stride[0] +
                         h * a.do_stride[2] + r * a.do_stride[1];
    const uint16_t* op = static_cast<const uint16_t*>(a.out) + b * a.o_stride[0] +
                         h * a.o_stride[2] + r * a.o_stride[1];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      df[k][c] = ld16(dp + 16 * c + 8 * lh);
      ov[k][c] = ld16(op + 16 * c + 8 * lh);
    }
  }
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    const int gw = gw0 + k;
    if (gw >= ntot) break;
    const int bh = gw / tiles;
    const int row = (gw % tiles) * 32 + lr;
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int w = 0; w < 4; ++w) part = T::dot2(ov[k][c][w], df[k][c][w], part);
    const float full = half_sum(part);
    if (row < Sq && lh == 0) {
      float* st = stats + 2 * (int64_t)bh * Sq;
      st[row] = (l[k] == neg_inf()) ? __builtin_inff() : l[k] * kLog2e;
      st[Sq + row] = full * a.softmax_scale;
    }
  }
}

// dQ = Σ_kb dS(qt, kb) K(kb) for head_dim 128 / 256 (dS carries the scale).  Workgroup: 8
// waves, wave w owns query tile qt = 8 qb + w of one query head; steps run
// over 32-key blocks.  Per step, wave w copies rows 4w..4w+3 of the K tile
// and its own 2 KB dS tile HBM -> LDS (buffer DMA: K rows past Sk and dS
// tiles past the wave's count read as zero), NBUF stages, NBUF - 1 in flight.
// Products (the layout of bwd_dq_kernel's dQᵀ += Kᵀ dSᵀ):
//   A = Kᵀ (d x key) by ds_read_b64_tr_b16 of the row-major K tile (16-byte
//       chunk swizzle of fa_fwd_d128.h), B = dSᵀ (key x query) by
//       ds_read_b64_tr_b16 of the dS tile.
// ds_read_b64_tr_b16 gives lane 16g + i, element j, element i%4 of the 8
// bytes read by lane 16g + 4j + i/4; both operands are read so that lane l
// gets keys 16kc + 8(l/32) + 4r + j (read r = 0, 1) of column l%32 (d for A,
// query for B).
template <int D>
struct DqDsShape {
  static constexpr int NW = 8;                   // (4: C2 71.4 against 68.2 us)
  static constexpr int RW = 32 / NW;             // K rows each wave copies per step
  static constexpr int ROWB = 2 * D;             // bytes per K row
  static constexpr int RPB = 1024 / ROWB;        // K rows per 1 KB DMA block
  static constexpr int CPR = D / 8;              // 16-byte chunks per row
  static constexpr int KBPW = RW / RPB;          // K blocks per wave and step
  // One workgroup per CU, four stages (three in flight).  head_dim 128, same
  // box, dQ kernel: C2 65.8 us against 77.4 (two workgroups per CU with three
  // stages each) and 68.3 (one with six); T1 within noise of both (418-435 us).
  static constexpr int NBUF = 4;
  static constexpr int WPE = 2;                  // waves per SIMD
  static constexpr int KTB = 32 * ROWB;          // K tile: 32 keys
  static constexpr int OFF_S = NBUF * KTB;       // dS stages after the K stages
  static constexpr int SSB = NW * 2048;          // dS stage: one tile per wave
  static constexpr int LDS = OFF_S + NBUF * SSB;
  static_assert((D == 128 || D == 256) && KBPW * RPB * NW == 32, "shape");
  static_assert(LDS * (WPE / 2) <= 160 * 1024, "LDS");
};

template <class T, int D, int MODE>
__global__ __launch_bounds__(64 * DqDsShape<D>::NW, DqDsShape<D>::WPE) void bwd_dq_ds_kernel(
    fa_bwd_args a, const uint16_t* ds) {
  using Sh = DqDsShape<D>;
  constexpr int NW = Sh::NW, ROWB = Sh::ROWB, NBUF = Sh::NBUF, KTB = Sh::KTB, KBPW = Sh::KBPW;
  constexpr int OFF_S = Sh::OFF_S, SSB = Sh::SSB;
  __shared__ __attribute__((aligned(16))) char smem[Sh::LDS];

  const int Sq = a.seqlen_q, Sk = a.seqlen_k, H = a.num_heads;
  const DsTiles L = ds_tiles<MODE>(Sq, Sk);
  const int nqb = (L.nq + NW - 1) / NW;
  const TileHead th = xcd_tile_order(blockIdx.x, nqb, a.batch * H);
  const int bh = th.bh, h = bh % H, b = bh / H;
  const int hk = h / (H / a.num_heads_k);
  // Causal: the longest query tiles (largest index) first.
  const int qb = MODE == kMaskCausal ? nqb - 1 - th.rank : th.rank;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 31, lh = lane >> 5;
  const int qt = NW * qb + wave;
  const int cnt = qt < L.nq ? L.count(qt) : 0;
  const int nsteps = L.count(min(NW * qb + NW - 1, L.nq - 1));

  // K rows 32s + 4w + rr, rr = RPB i + lane / CPR in block i, stored chunk
  // lane % CPR (logical chunk (lane % CPR) ^ swz(row), the swizzle acting on
  // the low four chunk bits); the lane's byte offset from the wave's first
  // row is fixed.
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[2];
  uint32_t k_loff[KBPW];
#pragma unroll
  for (int i = 0; i < KBPW; ++i) {
    const int rr = Sh::RPB * i + lane / Sh::CPR;
    k_loff[i] = 2u * (rr * (uint32_t)a.k_stride[1] +
                      8 * ((lane % Sh::CPR) ^ swz_chunk(Sh::RW * wave + rr)));
  }
  const uint16_t* ds_w =
      ds + 1024 * ((int64_t)bh * L.per_head() + L.prefix(min(qt, L.nq)));
  const u32x4 rs = rsrc_words(ds_w, (uint32_t)cnt * 2048u);
  // K resource of the next step to issue (steps are issued in order), based
  // at the wave's first row of that step and carried: one 64-bit add per
  // step; num_records covers RW rows except where they run past Sk.
  const uint32_t k_full = span_bytes(Sh::RW, a.k_stride[1], D);
  u32x4 rk = rsrc_words(kg + (int64_t)(Sh::RW * wave) * a.k_stride[1], k_full);
  const uint64_t k_step = 2ull * 32 * (uint64_t)a.k_stride[1];
  auto issue = [&](int s, int stage) {
    const int nb = 32 * s + Sh::RW * wave;
    u32x4 r = rk;
    if (nb + Sh::RW > Sk)
      r[2] = __builtin_amdgcn_readfirstlane(
          span_bytes(max(min(Sh::RW, Sk - nb), 0), a.k_stride[1], D));
#pragma unroll
    for (int i = 0; i < KBPW; ++i)
      buffer_lds16_opaque(r, k_loff[i], smem + stage * KTB + (KBPW * wave + i) * 1024);
    const uint64_t p = (((uint64_t)rk[1]) << 32 | rk[0]) + k_step;
    rk[0] = (uint32_t)p;
    rk[1] = (uint32_t)(p >> 32);
    buffer_lds16_stream2(rs, (uint32_t)s * 2048u + 16u * lane, smem + OFF_S + stage * SSB + wave * 2048);
  };

  // Transpose-read offsets.  A, read r, d tile dt: row 8(lane/32) + 4r +
  // (lane%16)/4 (+16 per key chunk: same swizzle), columns 32dt +
  // 16((lane/16)%2) + 4(lane%4).  B, read r: key 8(lane/32) + 4r + (lane%16)/4
  // (+16 per key chunk), half lane%2 and chunk kq = (lane/16)%2 of the
  // writer, i.e. row 16(lane/32) + 8(lane%2) + 4(r ^ kq) + (lane%16)/4 of
  // block kq (+32 rows = 512 bytes per key chunk), 8-byte half (lane%4)/2.
  int aoff[2][D / 32], boff[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int row = 8 * lh + 4 * r + ((lane & 15) >> 2);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      aoff[r][dt] = row * ROWB + 16 * (chunk ^ swz_chunk(row)) + 8 * (lane & 1);
    }
    const int kq = (lane >> 4) & 1;
    boff[r] = OFF_S + wave * 2048 + 1024 * kq +
              16 * (16 * lh + 8 * (lane & 1) + 4 * (r ^ kq) + ((lane & 15) >> 2)) +
              8 * ((lane & 3) >> 1);
  }

  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

  auto compute = [&](int stage) {
    const char* kt = smem + stage * KTB;
    const char* st = smem + stage * SSB;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const u32x2 b0 = lds_read_tr(st + boff[0] + 512 * kc);
      const u32x2 b1 = lds_read_tr(st + boff[1] + 512 * kc);
      const u32x4 bs = {b0[0], b0[1], b1[0], b1[1]};
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const u32x2 a0 = lds_read_tr(kt + aoff[0][dt] + 16 * ROWB * kc);
        const u32x2 a1 = lds_read_tr(kt + aoff[1][dt] + 16 * ROWB * kc);
        acc[dt] = T::mma32(u32x4{a0[0], a0[1], a1[0], a1[1]}, bs, acc[dt]);
      }
    }
  };

  // Step s: wait for this wave's DMAs of stage s (KBPW + 2 per stage; the
  // min(NBUF - 2, nsteps - 1 - s) stages after it stay in flight), barrier
  // (every wave's part of the K tile landed; the stage of step s - 1 is
  // free), refill that stage with step s + NBUF - 1.
  constexpr int PER_STAGE = KBPW + 2;
  static_assert(PER_STAGE == 3 || PER_STAGE == 4, "waits below");
  static_assert(NBUF == 4, "stage arithmetic and waits below");
  for (int s = 0; s < NBUF - 1 && s < nsteps; ++s) issue(s, s);
  auto step = [&](int s) {
    __syncthreads();
    if (s + NBUF - 1 < nsteps) issue(s + NBUF - 1, (s + NBUF - 1) & (NBUF - 1));
    if (s < cnt) compute(s & (NBUF - 1));
  };
  // All but the last two steps leave two stages in flight: one fixed wait.
  int s = 0;
  for (; s + 2 < nsteps; ++s) {
    __builtin_amdgcn_s_waitcnt(PER_STAGE == 3 ? 0x0F76 : 0x0F78);  // vmcnt(2 PER_STAGE)
    step(s);
  }
  for (; s < nsteps; ++s) {
    if (s + 1 < nsteps)
      __builtin_amdgcn_s_waitcnt(PER_STAGE == 3 ? 0x0F73 : 0x0F74);  // vmcnt(PER_STAGE)
    else
      wait_vmem();
    step(s);
  }
  wait_vmem();

  // acc[dt][4g + r] = dQ[32qt + lr][32dt + 8g + 4lh + r].
  const int row = 32 * qt + lr;
  if (qt >= L.nq || row >= Sq) return;
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
