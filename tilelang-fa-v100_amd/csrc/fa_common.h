// Shared device-side definitions for the gfx950 attention kernels.
//
// Conventions used by every kernel in this directory:
//  * A wavefront has 64 lanes.  `lane & 31` is written `lr` and `lane >> 5`
//    is written `lh`.
//  * The 32x32x16 MFMA (v_mfma_f32_32x32x16_{f16,bf16}) takes, per lane, an
//    8-element A vector holding A[row = lr][k = 8*lh + j] and an 8-element B
//    vector holding B[k = 8*lh + j][col = lr]; the 16 accumulators of a lane
//    hold C[row = 8*(i/4) + 4*lh + (i%4)][col = lr].
//    Because the hardware pairs A element (lane, j) with B element (lane, j),
//    any bijection from (lh, j) to the 16 k indices may be used as long as A
//    and B use the same one.  The kernels use that freedom so that the
//    accumulator of one product can be fed, without data movement, as the B
//    operand of the next one.
//  * 16-bit data are moved as raw 32-bit words (two elements per word, the
//    lower-indexed element in the low half).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#include "fa355.h"
#include "fa_tiles.h"

namespace fa {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4b __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Compile-time boolean tag (selects a code path through a generic lambda).
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};
// Compile-time integer tag.
template <int N>
struct IntC {
  static constexpr int value = N;
};

// Element-type traits.  `Half` is IEEE binary16, `BFloat16` is bfloat16.
struct Half {
  static constexpr int kId = 0;
  __device__ __forceinline__ static f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x4 mma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // 16x16x16: 4-element operands (k = 4 (lane / 16) + j).
  __device__ __forceinline__ static f32x4 mma16k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(
        __builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even conversion of two floats into one packed word.
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    f16x2 v;
    v[0] = (_Float16)lo;
    v[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  // Row-sum update for two probabilities p0, p1 whose packed form is w.
  // fp16 keeps 11 significant bits, so summing the rounded values (one
  // v_dot2_f32_f16 with ones) moves the LSE by at most 2^-11.  (The
  // ping-pong head_dim 128 core sums the fp32 values instead: there the
  // dot2 form overlaps the partner wave's matrix products worse.)
  __device__ __forceinline__ static float sum2(float, float, uint32_t w, float acc) {
    const f16x2 one = {(_Float16)1.f, (_Float16)1.f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
  }
  // acc + lo(a) lo(b) + hi(a) hi(b): the fp16 products are exact in fp32.
  __device__ __forceinline__ static float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc,
                                  false);
  }
  __device__ __forceinline__ static float lo(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, w)[0];
  }
  __device__ __forceinline__ static float hi(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, w)[1];
  }
};

struct BFloat16 {
  static constexpr int kId = 1;
  __device__ __forceinline__ static f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x4 mma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x4 mma16k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
        __builtin_bit_cast(s16x4b, a), __builtin_bit_cast(s16x4b, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    bf16x2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  // bf16 keeps 8 significant bits: the row sum uses the fp32 values.
  __device__ __forceinline__ static float sum2(float p0, float p1, uint32_t, float acc) {
    return acc + p0 + p1;
  }
  // acc + lo(a) lo(b) + hi(a) hi(b) in fp32 (exact products, two roundings).
  __device__ __forceinline__ static float dot2(uint32_t a, uint32_t b, float acc) {
    return fmaf(hi(a), hi(b), fmaf(lo(a), lo(b), acc));
  }
  __device__ __forceinline__ static float lo(uint32_t w) {
    return __builtin_bit_cast(float, w << 16);
  }
  __device__ __forceinline__ static float hi(uint32_t w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
  }
};

// acc += A·B on v_mfma_f32_32x32x16 with `acc` held in the accumulation
// registers (AGPRs) for its whole life.  For kernels whose accumulators fill
// the AGPR file next to a full VGPR file, the register allocator otherwise
// shuffles 16-register tuples between the two files and within the AGPRs
// (v_accvgpr_mov / read / write around every product).  The compiler's hazard
// pass does not look inside inline assembly, so the statement carries its
// own wait states: `s_nop 2` covers a VALU write of A or B just before it (2
// wait states are required); chained products on the same accumulator need
// none.  Callers publish zero-initialised accumulators to the asm with
// agpr_fence_in() and read results only after agpr_fence_out().
template <class T>
__device__ __forceinline__ void mma32_agpr(f32x16& acc, u32x4 a, u32x4 b) {
  if constexpr (T::kId == 0)
    asm("s_nop 2\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// After the VALU writes that initialise `acc` (2 wait states before an MFMA
// reads them as C).
__device__ __forceinline__ void agpr_fence_in(f32x16& acc) {
  asm volatile("s_nop 2" : "+a"(acc));
}
// Before any VALU read of `acc`: an 8- or 16-pass XDL write needs 11 or 19
// wait states before a VALU instruction reads the result.
__device__ __forceinline__ void agpr_fence_out(f32x16& acc) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(acc));
}

// Low 16 bits of `a` and of `b` packed as {a.lo, b.lo}; likewise for the high
// halves.  Used to transpose 16-bit matrices held in registers.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// Index of the calling wave in its workgroup, as a wave-uniform (scalar)
// value: branches on it then compile to scalar branches instead of EXEC
// masking with both paths issued.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// max / sum of x over lanes l and l ^ 32, in registers (no LDS round trip,
// whose lgkmcnt wait would also wait for LDS operand reads in flight).
// v_permlane32_swap swaps the upper 32 lanes of its first operand with the
// lower 32 lanes of its second; with x in both, lane l of the two results
// holds x[l] and x[l ^ 32], in an order that depends on the half, so only
// order-independent combinations are formed.  Inline assembly: the
// compiler folds the builtin's two results into one when both inputs are
// the same value.  `s_nop 1`: a VALU write of either operand needs 2 wait
// states before the swap reads it.
__device__ __forceinline__ void half_pair(float x, float& a, float& b) {
  a = x;
  b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float half_max(float x) {
  float a, b;
  half_pair(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float half_sum(float x) {
  float a, b;
  half_pair(x, a, b);
  return a + b;
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ u32x2 ld8(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ void st8(void* p, u32x2 v) {
  *reinterpret_cast<u32x2*>(p) = v;
}

// Visible (query i, key j) pairs of the dense paths: j <= i + off + wr when
// wr >= 0 and j >= i + off - wl when wl >= 0 (FlashAttention-2 window_size,
// causal is wr = 0), off = Sk - Sq.  Row / key bounds are checked separately.
struct Band {
  int off, wl, wr;
  // Some pair with i in [i0, i1] and j in [j0, j1] is inside the band.
  __device__ bool any(int i0, int i1, int j0, int j1) const {
    return (wr < 0 || j0 <= i1 + off + wr) && (wl < 0 || j1 >= i0 + off - wl);
  }
  // Every such pair is inside the band.
  __device__ bool all(int i0, int i1, int j0, int j1) const {
    return (wr < 0 || j1 <= i0 + off + wr) && (wl < 0 || j0 >= i1 + off - wl);
  }
  __device__ bool in(int i, int j) const {
    return (wr < 0 || j <= i + off + wr) && (wl < 0 || j >= i + off - wl);
  }
  // Query rows [first, end) that see any key in [j0, j1], clipped to [0, sq).
  __device__ int first_row(int j0) const { return wr >= 0 ? max(0, j0 - off - wr) : 0; }
  __device__ int end_row(int j1, int sq) const {
    return wl >= 0 ? min(sq, max(j1 - off + wl + 1, 0)) : sq;
  }
};

template <class Args>
__device__ __host__ __forceinline__ Band make_band(const Args& a) {
  const int wl = a.has_window ? a.window_left : -1;
  const int wr = a.causal ? 0 : (a.has_window ? a.window_right : -1);
  return Band{a.seqlen_k - a.seqlen_q, wl, wr};
}

// Mask variants a kernel is instantiated for.  kMaskCausal is the band
// wl = -1, wr = 0 and kMaskNone wl = wr = -1; building them from constants
// lets the compiler fold the window tests away (they cost registers in the
// hot loops).
enum MaskMode { kMaskNone = 0, kMaskCausal = 1, kMaskBand = 2 };

template <class Args>
__host__ __forceinline__ int mask_mode(const Args& a) {
  const Band b = make_band(a);
  if (b.wl < 0 && b.wr < 0) return kMaskNone;
  return (b.wl < 0 && b.wr == 0) ? kMaskCausal : kMaskBand;
}

template <int MODE, class Args>
__device__ __forceinline__ Band mode_band(const Args& a) {
  if constexpr (MODE == kMaskCausal) return Band{a.seqlen_k - a.seqlen_q, -1, 0};
  if constexpr (MODE == kMaskNone) return Band{a.seqlen_k - a.seqlen_q, -1, -1};
  return make_band(a);
}

// Butterfly reductions over the 64 lanes of a wave.
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}
__device__ __forceinline__ int wave_sum_int(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Epilogue of the forward cores for one valid row: the lane holds
// o[dt][4g + i] = O[row][32dt + 8g + 4lh + i] (unnormalised) and the row's
// sum l_all and base-2 running max ms_run.  Writes O / l_all to op in the
// input dtype and the natural-log LSE to lp (F32 false; lp nullptr: no LSE),
// or, for split-KV partials, O / l_all in fp32 and the base-2 LSE (F32
// true).  A row that saw no key gets O = 0 and LSE = -inf.
template <class T, bool F32, int DT>
__device__ __forceinline__ void fwd_store_ptrs(std::conditional_t<F32, float, uint16_t>* op,
                                               float* lp, int lh, const f32x16 (&o)[DT],
                                               float l_all, float ms_run) {
  const float inv = l_all > 0.f ? 1.f / l_all : 0.f;
  if constexpr (F32) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 w = {o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                         o[dt][4 * g + 3] * inv};
        *reinterpret_cast<f32x4*>(op + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) *lp = l_all > 0.f ? ms_run + log2f(l_all) : neg_inf();
  } else {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w[0] = T::pack(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv);
        w[1] = T::pack(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
        st8(op + 32 * dt + 8 * g + 4 * lh, w);
      }
    if (lp != nullptr && lh == 0) *lp = l_all > 0.f ? (ms_run + log2f(l_all)) * kLn2 : neg_inf();
  }
}

// The row's output pointers (fwd_store_ptrs) of problem P: O from column
// col0 on, and the LSE (nullptr when the problem stores none).
template <class Prob>
__device__ __forceinline__ auto fwd_out_ptr(const Prob& P, int row, int col0 = 0) {
  if constexpr (Prob::kF32Out)
    return P.o32_ptr(row) + col0;
  else
    return P.o_ptr(row) + col0;
}
template <class Prob>
__device__ __forceinline__ float* fwd_lse_ptr(const Prob& P, int row) {
  if constexpr (Prob::kF32Out)
    return P.lse2_ptr(row);
  else
    return P.has_lse ? P.lse_ptr(row) : nullptr;
}

// fwd_store_ptrs with the pointers formed from P at the store.
template <class T, int DT, class Prob>
__device__ __forceinline__ void fwd_store_row(const Prob& P, int row, int lh,
                                              const f32x16 (&o)[DT], float l_all,
                                              float ms_run, int col0 = 0) {
  fwd_store_ptrs<T, Prob::kF32Out>(fwd_out_ptr(P, row, col0), fwd_lse_ptr(P, row), lh, o, l_all,
                                   ms_run);
}

// Instruction-scheduling hint for a loop of N steps that each issue L LDS
// reads followed by M matrix products: the reads of the first `ahead` steps
// go first, then every step's products are followed by the reads of step
// + ahead.  Applies to the code emitted before it in the same basic block.
template <int N, int L, int M, int ahead>
__device__ __forceinline__ void sched_pipeline() {
  constexpr int kDsRead = 0x100, kMfma = 0x008;
  __builtin_amdgcn_sched_group_barrier(kDsRead, L * ahead, 0);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(kMfma, M, 0);
    if (i + ahead < N) __builtin_amdgcn_sched_group_barrier(kDsRead, L, 0);
  }
}

// Software pipeline of N steps whose operands come from LDS: the reads of
// step k + AHEAD are issued before the products of step k, with a
// scheduling barrier after every step, so AHEAD + 1 operand sets are live
// and each product waits only for its own reads (lgkmcnt of the later
// steps' reads).  load(k) returns step k's operands; use(k, ops) consumes
// them.  (The compiler's own scheduler, under register pressure, falls
// back to issuing each step's reads right before its products.)
template <int N, int AHEAD, class Load, class Use>
__device__ __forceinline__ void lds_pipeline(Load load, Use use) {
  using Ops = decltype(load(0));
  Ops ring[AHEAD + 1];
#pragma unroll
  for (int k = 0; k < AHEAD && k < N; ++k) ring[k] = load(k);
#pragma unroll
  for (int k = 0; k < N; ++k) {
    if (k + AHEAD < N) ring[(k + AHEAD) % (AHEAD + 1)] = load(k + AHEAD);
    use(k, ring[k % (AHEAD + 1)]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Buffer resources (gfx9 format): a 128-bit descriptor in scalar registers
// plus a 32-bit per-lane byte offset.  Accesses at offsets >= `bytes` are
// dropped (stores, atomics) or return zero (loads), which the kernels use to
// cut ragged tiles without branches.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcFlags);
}
// 16 bytes per lane from base + voff into LDS (lane l writes lds_block + 16l).
__device__ __forceinline__ void buffer_lds16(rsrc_t r, uint32_t voff, char* lds_block) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds_block, 16, voff, 0, 0, 0);
}
// 4 bytes per lane from base + voff into LDS (lane l writes lds_block + 4l).
__device__ __forceinline__ void buffer_lds4(rsrc_t r, uint32_t voff, void* lds_block) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds_block, 4, voff, 0, 0, 0);
}
// Bytes from the first of n rows (16-bit elements, `stride` elements apart)
// to the end of the last row's first `width` elements: the range of a buffer
// resource over those rows.  Rows past the n-th start at or beyond it when
// stride >= width; a size-1 dimension may carry stride 0, and then the range
// is still one row long.
__device__ __forceinline__ uint32_t span_bytes(int n, int64_t stride, int width) {
  return n > 0 ? 2u * ((uint32_t)(n - 1) * (uint32_t)stride + (uint32_t)width) : 0u;
}
// Buffer descriptor words for the inline-assembly DMA below (same fields as
// make_rsrc: raw buffer, stride 0, num_records = bytes).
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, bytes, (uint32_t)kRsrcFlags};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// LDS DMA the compiler does not see: buffer_lds16 / a 4-byte global_load_lds
// issued from inline assembly.  The compiler treats every LDS access after a
// DMA it knows of as possibly aliasing the DMA target unless it can prove
// otherwise, and then waits for vmcnt(0) - which also waits for every
// other outstanding global load.  With these forms the caller owns the wait:
// wait_vmem() before any wave reads the target (followed by a barrier when
// other waves read it).  M0 (the LDS base of the DMA) is a register the
// compiler reserves, so the statements save it and put it back.
__device__ __forceinline__ void buffer_lds16_opaque(u32x4 rsrc, uint32_t voff, char* lds_block) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(lds_addr(lds_block))
      : "memory");
}
// Four buffer_lds16_opaque DMAs from one resource (lane offsets v0..v3)
// into the consecutive 1 KB blocks from lds_block on: one M0 value, stepped
// by 1 KB between the instructions.  With one M0 value per block the
// compiler held all of them (four per DMA site) in scalar registers and
// spilled them; each DMA in the forward key loop then reloaded its M0 with a
// v_readlane.
__device__ __forceinline__ void buffer_lds16_x4(u32x4 rsrc, uint32_t v0, uint32_t v1, uint32_t v2,
                                                uint32_t v3, const char* lds_block) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %6\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %5, 0 offen lds\n\t"
      "s_add_u32 m0, m0, 0x400\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %5, 0 offen lds\n\t"
      "s_add_u32 m0, m0, 0x400\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %3, %5, 0 offen lds\n\t"
      "s_add_u32 m0, m0, 0x400\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %4, %5, 0 offen lds\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(v0), "v"(v1), "v"(v2), "v"(v3), "s"(rsrc), "s"(lds_addr(lds_block))
      : "scc", "memory");
}
// Two buffer_lds16_opaque DMAs from two resources: (r0, v0) into lds_block
// and (r1, v1) into lds_block + STEP, under one saved M0.
template <int STEP>
__device__ __forceinline__ void buffer_lds16_pair(u32x4 r0, uint32_t v0, u32x4 r1, uint32_t v1,
                                                  const char* lds_block) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %5\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_add_u32 m0, m0, %6\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %3, %4, 0 offen lds\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(v0), "s"(r0), "v"(v1), "s"(r1), "s"(lds_addr(lds_block)), "i"(STEP)
      : "scc", "memory");
}
__device__ __forceinline__ void global_lds4_opaque(const void* src, void* lds_block) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds_addr(lds_block))
      : "memory");
}

// 16 bytes per lane from src into LDS (lane l writes lds_block + 16l), as an
// opaque global_load_lds_dwordx4 (same contract as global_lds4_opaque).  With
// the compiler-visible form the waitcnt pass counted every later LDS read
// against the DMA and waited for lgkmcnt(0) before each product, so operand
// reads issued ahead of a product gave no overlap.
__device__ __forceinline__ void global_lds16_opaque(const void* src, void* lds_block) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds_addr(lds_block))
      : "memory");
}

// Workgroup order for a grid of ntiles x nbh tiles (nbh = batch x heads).
// The hardware hands workgroup ids to the 8 XCDs round-robin and each XCD
// starts its ids in increasing order.  Each XCD is given a contiguous block
// of heads (tiles of one head share K/V or Q/dO in that XCD's L2), and within
// its heads it starts every head's rank-0 tile, then every rank-1 tile, and
// so on; with rank 0 the most expensive causal tile, long tiles start first
// and short ones fill the tail.  Falls back to rank-major over all heads when
// nbh is not a multiple of 8.
struct TileHead {
  int rank, bh;
};
__device__ __forceinline__ TileHead xcd_tile_order(int wg, int ntiles, int nbh) {
  constexpr int kXcds = 8;
  if (nbh % kXcds == 0) {
    const int per = nbh / kXcds;
    const int local = wg / kXcds;
    return {local / per, (wg % kXcds) * per + local % per};
  }
  return {wg / nbh, wg % nbh};
}

// Persistent schedule over the virtual workgroup ids of xcd_tile_order: a
// grid of W workgroups (as many as fit the GPU at once) walks total =
// ntiles x nbh tiles, workgroup w taking one tile per round r.  Within a
// round the tiles go out in xcd_tile_order's order (heaviest causal rank
// first), and the direction alternates between rounds (the heaviest tile of
// one round pairs with the lightest of the next), which balances the
// per-workgroup sums of linearly decreasing tile costs.  When nbh is a
// multiple of 8 (then W is too), workgroup w stays on its XCD's heads: it
// runs on XCD w % 8 and takes virtual ids 8 local + w % 8.  Returns the
// virtual id, or -1 when workgroup w has no tile in round r (nor in any
// later round).
__device__ __forceinline__ int persistent_tile(int w, int W, int r, int total, int nbh) {
  constexpr int kXcds = 8;
  if (nbh % kXcds == 0) {
    const int wx = W / kXcds, l = w / kXcds;
    const int local = r * wx + ((r & 1) ? wx - 1 - l : l);
    return local < total / kXcds ? local * kXcds + w % kXcds : -1;
  }
  const int v = r * W + ((r & 1) ? W - 1 - w : w);
  return v < total ? v : -1;
}

// The kernel's arguments, read through a pointer the compiler cannot
// follow, so each use reloads them from the kernarg segment (scalar loads)
// instead of keeping every field in scalar registers for the kernel's whole
// life: a persistent loop that sets up each tile from them would otherwise
// spill.
template <class Args>
__device__ __forceinline__ const __attribute__((address_space(4))) Args* kernel_args() {
  auto p = (const __attribute__((address_space(4))) Args*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return p;
}

// XCD-aware workgroup order.  The hardware hands consecutive workgroup ids to
// the 8 XCDs round-robin; remapping makes each XCD receive a contiguous range
// of logical tiles, so tiles that share K/V rows share one L2.
__device__ __forceinline__ int xcd_remap(int linear, int total) {
  constexpr int kXcds = 8;
  if (total % kXcds != 0) return linear;
  const int per = total / kXcds;
  return (linear % kXcds) * per + linear / kXcds;
}

}  // namespace fa
