// Paged decode for gfx950: split-KV partials + LSE-merge combine.
//
// Replaces _decode_kernel_func (tilelang_fa_v100/_kernels_paged.py:393-489),
// which runs one workgroup per (query head, sequence), walks the whole
// context serially and re-reads every KV head once per query head.  Here a
// workgroup owns (fixed-size key chunk, KV head, head group, sequence):
//   * all GB query heads of a GQA group are served by one read of the chunk's
//     K and V rows (GB = largest of 8/4/2/1 dividing Hq/Hkv);
//   * every K and V load of the chunk is issued first (16 + 16 vectors of
//     16 bytes per lane), so a workgroup keeps its whole chunk in flight;
//   * phase 1: S^T = K Q^T on the 16x16x32 MFMA (A = K rows from the paged
//     cache in registers; B = Q^T, unused head columns zero);
//   * phase 2: per-head max / exp2 / sum over the chunk in LDS;
//   * phase 3: O += P V on the VALU, each lane owning 8 contiguous d of a V
//     row, followed by a cross-lane and cross-wave reduction;
//   * each chunk writes a normalised partial O (fp32) and its base-2 LSE; the
//     combine kernel merges chunks with LSE weights (the online-softmax merge
//     of the dormant split variant, _kernels_paged.py:175-187).
// The decode mask is `key < seq_len` (_kernels_paged.py:450-451).
#include <algorithm>
#include <mutex>

#include "fa_common.h"
#include "fa_decode_stream.h"
#include "fa_internal.h"

namespace fa {

// Keys per split workgroup: every lane then holds 16 K and 16 V vectors of
// 16 bytes (32768 / D keys for any D), all loads issued before any use.
template <int D>
struct DecShape {
  static constexpr int CH = tiles::kDecChunkElems / D;  // keys per chunk (256 for D=128)
  static constexpr int DC = D / 32;      // 32-wide d chunks of the QK^T MFMA
  static constexpr int KIT = CH / 64;    // 16-key blocks per wave (phase 1)
  static constexpr int LPT = D / 8;      // lanes per V row (phase 3)
  static constexpr int TPW = 64 / LPT;   // V rows per wave per pass
  static constexpr int TPB = 4 * TPW;    // V rows per workgroup per pass
  static constexpr int VIT = CH / TPB;   // passes (phase 3)
  static_assert(KIT * DC == 16 && VIT == 16, "16 K and 16 V loads per lane");
};

__host__ __device__ constexpr int dec_chunk(int D) { return tiles::kDecChunkElems / D; }

struct DecodeWs {
  float* po;    // [B, Hq, nsplit, D]   normalised partial outputs
  float* plse;  // [B, Hq, nsplit]      base-2 log-sum-exp of each chunk
  int nsplit;
  int split;       // keys per split
  int* split_dev;  // when set, the split size used is read here (the streaming kernel's)
};

template <class T, int D, int GB>
__global__ __launch_bounds__(256, 2) void decode_split_kernel(fa_decode_args a,
                                                              DecodeWs ws) {
  using S = DecShape<D>;
  constexpr int CH = S::CH;
  __shared__ __attribute__((aligned(16))) float s_lds[GB][CH];
  __shared__ float red[4][GB][D];
  __shared__ float stat_m[GB], stat_l[GB];

  const int G = a.num_heads / a.num_kv_heads;
  const int ngroups = G / GB;
  const int id = blockIdx.x;
  const int c = id % ws.nsplit;
  int rest = id / ws.nsplit;
  const int hg = rest % ngroups;
  rest /= ngroups;
  const int hk = rest % a.num_kv_heads;
  const int b = rest / a.num_kv_heads;

  const int seq_len = max(0, min(a.seq_lens[b], a.max_blocks * a.page_size));
  const int n_begin = c * CH;
  if (n_begin >= seq_len) return;
  const int n_end = min(n_begin + CH, seq_len);
  const int n_last = n_end - 1;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int h0 = hk * G + hg * GB;  // first query head of this group
  const uint16_t* kc = static_cast<const uint16_t*>(a.k_cache) + (int64_t)hk * a.k_stride[2];
  const uint16_t* vc = static_cast<const uint16_t*>(a.v_cache) + (int64_t)hk * a.v_stride[2];
  const int32_t* bt = a.block_table + (int64_t)b * a.block_table_stride;
  const int ps_log2 = __builtin_ctz(a.page_size);
  const int ps_mask = a.page_size - 1;
  const unsigned last_page = (unsigned)(a.num_pages - 1);
  // Keys past the chunk end are read from its last key (finite data that is
  // masked or multiplied by P = 0), so every load is unconditional.
  auto row_of = [&](const uint16_t* base, int64_t page_stride, int64_t slot_stride,
                    int n) -> const uint16_t* {
    n = min(n, n_last);
    const int64_t page = (int64_t)min((unsigned)bt[n >> ps_log2], last_page);
    return base + page * page_stride + (n & ps_mask) * slot_stride;
  };
  const float scale_log2 = a.softmax_scale * kLog2e;

  // ---- issue every load of the chunk: K in MFMA-A layout, V rows for phase 3.
  const int l16 = lane & 15, lq = lane >> 4;
  const int lsub = lane % S::LPT, lrow = lane / S::LPT;
  u32x4 kr[S::KIT][S::DC], vr[S::VIT];
#pragma unroll
  for (int it = 0; it < S::KIT; ++it) {
    const uint16_t* kp = row_of(kc, a.k_stride[0], a.k_stride[1],
                                n_begin + (wave + 4 * it) * 16 + l16);
#pragma unroll
    for (int cc = 0; cc < S::DC; ++cc) kr[it][cc] = ld16(kp + 32 * cc + 8 * lq);
  }
#pragma unroll
  for (int it = 0; it < S::VIT; ++it) {
    const uint16_t* vp = row_of(vc, a.v_stride[0], a.v_stride[1],
                                n_begin + it * S::TPB + wave * S::TPW + lrow);
    vr[it] = ld16(vp + 8 * lsub);
  }

  // ---- phase 1: S^T = K Q^T on the 16x16x32 MFMA (columns = query heads).
  {
    u32x4 qb[S::DC];
    const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_stride[0] +
                           (int64_t)(h0 + min(l16, GB - 1)) * a.q_stride[1];
#pragma unroll
    for (int cc = 0; cc < S::DC; ++cc) {
      const u32x4 qv = ld16(qrow + 32 * cc + 8 * lq);
      qb[cc] = (l16 < GB) ? qv : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int it = 0; it < S::KIT; ++it) {
      const int blk = wave + 4 * it;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < S::DC; ++cc) acc = T::mma16(kr[it][cc], qb[cc], acc);
      // acc[i] = S^T[key = blk*16 + 4*lq + i][head = l16]
      if (l16 < GB) {
        f32x4 sv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int nn = n_begin + blk * 16 + 4 * lq + i;
          sv[i] = nn < n_end ? acc[i] * scale_log2 : neg_inf();
        }
        *reinterpret_cast<f32x4*>(&s_lds[l16][blk * 16 + 4 * lq]) = sv;
      }
    }
  }
  __syncthreads();

  // ---- phase 2: per-head max and sum (base 2).
  for (int g = wave; g < GB; g += 4) {
    float m = neg_inf();
    for (int t = lane; t < CH; t += 64) m = fmaxf(m, s_lds[g][t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < CH; t += 64) {
      const float p = fast_exp2(s_lds[g][t] - m);
      s_lds[g][t] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      stat_m[g] = m;
      stat_l[g] = l;
    }
  }
  __syncthreads();

  // ---- phase 3: O = P V on the VALU, 8 d per lane.
  float acc[GB][8];
#pragma unroll
  for (int g = 0; g < GB; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
#pragma unroll
  for (int it = 0; it < S::VIT; ++it) {
    const int t = it * S::TPB + wave * S::TPW + lrow;
    float vf[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      vf[2 * w] = T::lo(vr[it][w]);
      vf[2 * w + 1] = T::hi(vr[it][w]);
    }
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      const float p = s_lds[g][t];  // 0 for keys past the chunk end
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(p, vf[j], acc[g][j]);
    }
  }
  // Reduce over the key rows held by lanes of equal lsub within the wave.
#pragma unroll
  for (int o = S::LPT; o < 64; o <<= 1)
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] += __shfl_xor(acc[g][j], o);
  if (lrow == 0) {
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[wave][g][8 * lsub + j] = acc[g][j];
  }
  __syncthreads();
  for (int e = tid; e < GB * D; e += 256) {
    const int g = e / D, d = e % D;
    const float sum = red[0][g][d] + red[1][g][d] + red[2][g][d] + red[3][g][d];
    const float l = stat_l[g];
    const int64_t row = ((int64_t)b * a.num_heads + h0 + g) * ws.nsplit + c;
    ws.po[row * D + d] = l > 0.f ? sum / l : 0.f;
    if (d == 0) ws.plse[row] = l > 0.f ? stat_m[g] + log2f(l) : neg_inf();
  }
}

// One wave per (sequence, query head): merge the chunk partials with weights
// exp2(lse_c - max), computed lane-parallel, then an unrolled weighted sum.
template <class T, int D>
__global__ __launch_bounds__(64) void decode_combine_kernel(fa_decode_args a,
                                                            DecodeWs ws) {
  const int CH = ws.split_dev ? *ws.split_dev : ws.split;
  constexpr int NP = (D + 127) / 128;  // d pairs per lane: 2*lane + 128*k
  __shared__ float wts[64];
  const int hq = blockIdx.x % a.num_heads;
  const int b = blockIdx.x / a.num_heads;
  const int lane = threadIdx.x;
  const int seq_len = max(0, min(a.seq_lens[b], a.max_blocks * a.page_size));
  const int ns = (seq_len + CH - 1) / CH;
  const int64_t row0 = ((int64_t)b * a.num_heads + hq) * ws.nsplit;
  float m = neg_inf();
  for (int c = lane; c < ns; c += 64) m = fmaxf(m, ws.plse[row0 + c]);
  m = wave_max(m);
  const float m_use = (m == neg_inf()) ? 0.f : m;
  float acc[NP][2];
#pragma unroll
  for (int k = 0; k < NP; ++k) acc[k][0] = acc[k][1] = 0.f;
  float wsum = 0.f;
  for (int c0 = 0; c0 < ns; c0 += 64) {
    const int cn = min(64, ns - c0);
    const float w = lane < cn ? fast_exp2(ws.plse[row0 + c0 + lane] - m_use) : 0.f;
    wsum += wave_sum(w);
    wts[lane] = w;
    __syncthreads();
    const float* base = ws.po + (row0 + c0) * D;
#pragma unroll 8
    for (int c = 0; c < cn; ++c) {
      const float wc = wts[c];
#pragma unroll
      for (int k = 0; k < NP; ++k) {
        const int d = 2 * lane + 128 * k;
        if (d < D) {
          const float2 pv = *reinterpret_cast<const float2*>(base + (int64_t)c * D + d);
          acc[k][0] = fmaf(wc, pv.x, acc[k][0]);
          acc[k][1] = fmaf(wc, pv.y, acc[k][1]);
        }
      }
    }
    __syncthreads();
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  uint16_t* op = static_cast<uint16_t*>(a.out) + (int64_t)b * a.o_stride[0] +
                 (int64_t)hq * a.o_stride[1];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int d = 2 * lane + 128 * k;
    if (d < D)
      *reinterpret_cast<uint32_t*>(op + d) = T::pack(acc[k][0] * inv, acc[k][1] * inv);
  }
  if (a.lse && lane == 0)
    a.lse[(int64_t)b * a.num_heads + hq] =
        wsum > 0.f ? (m_use + log2f(wsum)) * kLn2 : neg_inf();
}

// ----------------------------------------------------------------- launchers

int decode_group_size(const fa_decode_args& a) {
  const int G = a.num_heads / a.num_kv_heads;
  if (G % 8 == 0) return 8;
  if (G % 4 == 0) return 4;
  if (G % 2 == 0) return 2;
  return 1;
}

// The streaming kernel (fa_decode_stream.h) covers head_dim 64 - 512 with
// pages of at least 16 keys, or of at least the 1024 / 2D rows one of its
// DMA instructions loads (8 keys at head_dim 64, 4 at 128, 2 at 256, 1 at
// 512), at most kMaxGroup query heads per item and token strides whose
// 16-row offsets fit its 32-bit lane offsets; other shapes use
// decode_split_kernel.
static bool use_stream(const fa_decode_args& a) {
  const int64_t lim = int64_t(1) << 26;
  return (a.page_size >= 16 || a.page_size * 2 * a.head_dim >= 1024) &&
         a.batch <= DecStream<128>::kMaxBatch &&
         decode_group_size(a) <= DecStream<128>::kMaxGroup && a.k_stride[1] >= 0 &&
         a.k_stride[1] < lim && a.v_stride[1] >= 0 && a.v_stride[1] < lim;
}

// Resident waves per CU of the streaming kernel for head_dim D.
static int stream_waves_per_cu(int D) {
  switch (D) {
    case 64: return DecStream<64>::kWavesPerCU;
    case 256: return DecStream<256>::kWavesPerCU;
    case 512: return DecStream<512>::kWavesPerCU;
  }
  return DecStream<128>::kWavesPerCU;
}

// Keys per split.  The streaming kernel takes the largest of kSplitMax,
// kSplitMax / 2, .. kSplitMin whose item count (estimated from max_seq_len)
// gives every resident wave at least kDecItemsPerWave items.
static int decode_split_size(const fa_decode_args& a) {
  if (!use_stream(a)) return dec_chunk(a.head_dim);
  const int G = a.num_heads / a.num_kv_heads;
  const int64_t heads = (int64_t)a.num_kv_heads * (G / decode_group_size(a));
  const int64_t waves = (int64_t)device_cu_count() * stream_waves_per_cu(a.head_dim);
  int s = tiles::kDecSplitKeysMax;
  for (; s > tiles::kDecSplitKeysMin; s /= 2) {
    const int64_t items = (int64_t)a.batch * ((a.max_seq_len + s - 1) / s) * heads;
    if (items >= tiles::kDecItemsPerWave * waves) break;
  }
  return s;
}

int decode_num_splits(const fa_decode_args& a) {
  const int ch = decode_split_size(a);
  return (a.max_seq_len + ch - 1) / ch;
}


size_t decode_workspace_bytes(const fa_decode_args& a) {
  const size_t rows = (size_t)a.batch * a.num_heads * (size_t)decode_num_splits(a);
  return rows * (size_t)a.head_dim * sizeof(float) + rows * sizeof(float) + 256;
}

// Queried once per device (std::call_once: entry points may run on several
// host threads at once).
int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::once_flag once[kMaxDevices];
  static int cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  });
  return cached[dev];
}

template <class T, int D>
static hipError_t launch_combine(const fa_decode_args& a, DecodeWs ws, hipStream_t st) {
  hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3((unsigned)(a.batch * a.num_heads)),
                     dim3(64), 0, st, a, ws);
  return hipGetLastError();
}

template <class T, int D, int GB>
static hipError_t launch_decode_gb(const fa_decode_args& a, DecodeWs ws,
                                   hipStream_t st) {
  const int G = a.num_heads / a.num_kv_heads;
  const int64_t items = (int64_t)ws.nsplit * (G / GB) * a.num_kv_heads * a.batch;
  if (items > 0) {  // max_seq_len == 0: the combine alone writes zeros
    if (use_stream(a)) {
      using SD = DecStream<D>;
      const int64_t wgs = std::max<int64_t>(
          1, std::min<int64_t>((items + SD::kWavesPerWG - 1) / SD::kWavesPerWG,
                               (int64_t)device_cu_count() * SD::kWavesPerCU / SD::kWavesPerWG));
      DecodeWsS wss{ws.po, ws.plse, ws.split_dev, ws.nsplit, ws.split};
      hipLaunchKernelGGL((decode_stream_kernel<T, SD::D, GB>), dim3((unsigned)wgs),
                         dim3(64 * SD::kWavesPerWG), 0, st, a, wss);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      return launch_combine<T, D>(a, ws, st);
    }
    ws.split_dev = nullptr;  // the chunked kernel uses the launcher's split
    hipLaunchKernelGGL((decode_split_kernel<T, D, GB>), dim3((unsigned)items), dim3(256), 0, st,
                       a, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_combine<T, D>(a, ws, st);
  }
  // No split kernel ran, so no split size was recorded on the device.
  ws.split_dev = nullptr;
  return launch_combine<T, D>(a, ws, st);
}

template <class T, int D>
static hipError_t launch_decode_d(const fa_decode_args& a, DecodeWs ws, hipStream_t st) {
  switch (decode_group_size(a)) {
    case 8: return launch_decode_gb<T, D, 8>(a, ws, st);
    case 4: return launch_decode_gb<T, D, 4>(a, ws, st);
    case 2: return launch_decode_gb<T, D, 2>(a, ws, st);
    default: return launch_decode_gb<T, D, 1>(a, ws, st);
  }
}

template <class T>
static hipError_t launch_decode_t(const fa_decode_args& a, DecodeWs ws, hipStream_t st) {
  switch (a.head_dim) {
    case 64: return launch_decode_d<T, 64>(a, ws, st);
    case 128: return launch_decode_d<T, 128>(a, ws, st);
    case 256: return launch_decode_d<T, 256>(a, ws, st);
    case 512: return launch_decode_d<T, 512>(a, ws, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_decode(const fa_decode_args& a, void* workspace, hipStream_t st) {
  DecodeWs ws;
  ws.nsplit = decode_num_splits(a);
  ws.split = decode_split_size(a);
  const size_t rows = (size_t)a.batch * a.num_heads * (size_t)ws.nsplit;
  char* base = static_cast<char*>(workspace);
  ws.po = reinterpret_cast<float*>(base);
  ws.plse = reinterpret_cast<float*>(base + rows * a.head_dim * sizeof(float));
  // One int after the partial LSEs (inside the workspace's 256-byte tail).
  ws.split_dev = reinterpret_cast<int*>(ws.plse + rows);
  return a.dtype == FA_DTYPE_BF16 ? launch_decode_t<BFloat16>(a, ws, st)
                                  : launch_decode_t<Half>(a, ws, st);
}

}  // namespace fa
