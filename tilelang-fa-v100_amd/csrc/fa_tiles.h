// Fixed gfx950 tile table.
//
// Replaces the reference's run-time autotuner (tilelang_fa_v100/_configs.py:5-79
// candidate generators, _utils.py:4-27 SM70 validity model, the fixed
// _BEST_CONFIGS / _DECODE_BEST_CONFIGS dicts in _kernels_paged.py:353-364,
// 495-499).  Every kernel takes its tile sizes from here; nothing is tuned at
// run time, so the first call of a shape costs no compilation or search.
// Each entry states the measurement (MI355X, rocprofv3 counters or event
// timing of T1 = causal fp16 B=2 S=8192 H=16 D=128, C2 = the same at B=4
// S=2048) that chose it over the alternatives tried.
#pragma once

namespace fa {
namespace tiles {

// ---- dense / paged forward, head_dim 128 (fa_fwd_d128.h)
// 256 query rows per workgroup = 8 waves x 32 rows (two waves per SIMD, 207
// VGPRs, no spills), 64-key K/V tiles double-buffered in LDS (64 KB).
// Evidence: T1 forward 0.545 ms, MFMA busy 52.5% (SQ_VALU_MFMA_BUSY_CYCLES);
// 4-wave / 128-row workgroups (two per CU) measured 0.673 ms against 0.640 ms
// for this shape under the same (one-phase) schedule; LDS bank conflicts 0
// (SQ_LDS_BANK_CONFLICT) with the 16-byte chunk swizzle.
constexpr int kFwd128Rows = 256;
constexpr int kFwd128Keys = 64;
constexpr int kFwd128Waves = 8;

// ---- dense / paged forward, head_dim 256 (fa_fwd_1w.h)
// 4 waves x 32 rows, one wave per SIMD, one pass over 32-key tiles with O in
// AGPRs (256 VGPRs + 155 AGPRs, no spills).  Evidence, T1 shape at head_dim
// 256 (B=2, S=8192, H=8, causal), same box: 0.638-0.649 ms against
// 0.760-0.763 ms for 8 waves x 32 rows at two waves per SIMD (230 VGPRs, O in
// two 128-column passes with the scores recomputed, 1.5x the products),
// bit-identical outputs; that schedule in turn took 0.844 ms against 1.204 ms
// for the one-pass register-staged 4-wave core (406 registers, accumulators
// shuffled between the register files).
constexpr int kFwd256Rows = 128;

// ---- forward, head_dim 64 / 256 / 512 (fa_fwd_core.h; head_dim 256 only for
// paged problems with pages of fewer than 16 keys)
// 128 query rows per workgroup (4 waves x 32 rows); keys per tile
// 8192 / D for D <= 256 (a 16 KB K tile), 32 for D = 512, whose O columns are
// accumulated in two 256-wide passes so Q, O and the staging fit one wave's
// 512 registers; 2 waves per SIMD for D <= 128, 1 above.
// Evidence (compiler resource usage): D = 64 takes 182 VGPRs and D = 256
// 254 VGPRs + 152 AGPRs (one wave per SIMD), both without spills; D = 512
// (two O passes) 253 VGPRs + 160 AGPRs in the VGPR MFMA form fa_fwd.hip is
// built in (35 spilled in the default form).  Dense problems too small to
// give half the CUs a 128-row tile (C1) take the key-split kernel below.
constexpr int kFwdCoreRows = 128;
constexpr int kFwdCoreTileElems = 8192;  // keys x head_dim per K tile (D <= 256)
constexpr int kFwdCoreKeys512 = 32;

// ---- dense forward with keys split across the waves of a workgroup
// (fa_fwd_split.h), head_dim 64 / 128: used when the standard cores' grid
// would give fewer than a kFwdSplitMaxFill share of the CUs a workgroup
// (configs[0], [1, 512, 16, 64]: 64 workgroups of 128 rows for 256 CUs).
// 32 query rows per workgroup; 8 waves (two per SIMD), each with a private
// pair of 32-key K / V tiles (double-buffered at head_dim 64, single at 128;
// 128 KB of LDS).  Evidence (event time per call, same box): C1 9.2 us
// against 13.5 us on the 128-row core (kernel trace 7.4 against 12.5 us) and
// 10.9 us with 16 waves (one tile each, single-buffered); [1, 2048, 8, 128]
// 43.0 / 33.2 us (full / causal) against 47.8 / 36.6 us with 4 waves and
// 57.4 / 55.0 us on the 256-row core; [4, 300, 8, 128] 18.6 us against 16.6
// (4 waves) and 18.9 (256-row core).
constexpr int kFwdSplitWaves64 = 8;
constexpr int kFwdSplitWaves128 = 8;
constexpr int kFwdSplitMaxFillNum = 1, kFwdSplitMaxFillDen = 2;  // one half

// ---- backward dK / dV kernel, head_dim 128 / 256 (fa_bwd_mfma.h)
// KV-stationary: head_dim 128 keeps 256 keys per workgroup (8 waves x 32 keys,
// dK / dV of a wave's 32 keys in 128 registers), head_dim 256 keeps 128 keys
// (4 waves); 32 query rows per iteration.  Evidence: every Q / dO tile read
// from LDS serves the whole key tile, so the largest key tile whose dK / dV fit
// the register file wins; 4 waves x 64 keys (512 registers each) measured
// 2.31 ms against 1.81 ms (T1 backward), and a two-group ping-pong schedule
// with three Q / dO buffers 1.115 against 1.105 ms for the kernel (it runs
// near the LDS read rate: five 1 KB operand reads per four MFMAs).
constexpr int kBwdQueryRows = 32;
// Measured again with the current kernel (same box, T1 backward, dK / dV /
// dQ bit-identical in every variant): 4 waves x 64 keys at one wave per SIMD
// (dK / dV of 64 keys pinned in the 256 AGPRs, every Q / dO / Qᵀ / dOᵀ read
// feeding two products) 1.85 ms against 1.69-1.77 ms for 8 waves x 32 keys,
// and C2 0.29 against 0.26-0.27 ms.  Counters (T1): the same MFMA busy
// cycles but co-execution of MFMA and VALU 10x lower (3.0e7 against 2.9e8
// cycles): a lone wave issues in order, so its softmax runs between its
// products instead of under the partner wave's.  Interleaving the element
// work into the chains (exponentials between the dP products, dS between the
// dV products, separate S / dP / dV / dK chains) compiled without spills
// only with the masked / unmasked branch confined to the element work, and
// still measured 1.81-1.93 ms (head_dim 256, same schedule: 1.76-1.87
// against 1.64-1.70 ms for the combined S / dP loop and dV / dK chain).

// ---- backward: dQ (fa_bwd_dq.h), query-stationary, no atomics.  Evidence
// (fa_bwd per call, ms, dQ by fp32 atomics from the key-stationary kernel /
// query-stationary kernel, fp16): D=64 B4 S2048 H16 causal 0.405 / 0.343,
// full 0.523 / 0.443; D=128 C2 causal 0.314 / 0.300, full 0.521 / 0.507, T1
// 1.811 / 1.814, GQA 32/8 B2 S4096 causal 1.283 / 1.224, full 1.733 / 1.772,
// B1 S16384 H8 1.767 / 1.777, B8 S1024 0.203 / 0.208; D=256 B2 S8192 H8 causal
// 3.474 / 2.409 (with fa_bwd.hip compiled for VGPR-form MFMA, see build.py).
// The atomics are performed beyond the XCD's L2 on this part, ~64 address
// cycles per instruction, a floor of ~1.17 ms for T1's backward.

// ---- backward: dQ from stored dS tiles (fa_bwd_ds.h), head_dim 128 / 256,
// causal or full attention, while the tiles (2 bytes per visible (query, key)
// pair, 2.15 GB at T1) stay within this many bytes; larger problems recompute
// S and dP in bwd_dq_kernel.
constexpr size_t kBwdDsMaxBytes = size_t(4) << 30;

// ---- backward main kernel, head_dim 64 (fa_bwd.hip)
// 128 keys per workgroup, 64 query rows per iteration, 4 waves.
constexpr int kBwd64Keys = 128;
constexpr int kBwd64QueryRows = 64;

// ---- decode, head_dim 64 / 128 / 256 / 512, pages of at least 16 keys or of
// at least one DMA instruction's 1024 / 2D rows (fa_decode_stream.h)
// Persistent waves; work item = a split of keys x one KV head x its query
// heads (up to 8, the 16x16x32 MFMA columns); 16-key tiles, two in flight
// per wave.  Keys per split: the largest of kDecSplitKeysMax, /2, /4 ..
// kDecSplitKeysMin whose item count, estimated from max_seq_len, is at least
// kDecItemsPerWave per resident wave (long items amortise each item's query
// load and partial-result store; enough items keep every wave streaming);
// the kernel doubles it when the actual lengths allow (T2 83%, C4 stays 80%).
// Evidence (C4 = 64 sequences of 1083-32645 keys, T2 = 64 x 32768; % of
// 8 TB/s, cache flushed by a read): split 256: 67.6 / 66.8; 512: 71.3 /
// 74.1; 1024: 75.3 / 76.3; 2048: 79.5 / 80.9; 4096: 66.2 / 83.4 (C4 then
// has ~1 item per wave, and max_seq_len cannot tell it from T2).  T2 reads
// 1.006x its algorithmic bytes (FETCH_SIZE).  Head_dim 64 and 256 run the same
// kernel with the ring depth and waves per workgroup scaled so that every CU
// keeps ~128 KB of K / V in flight (64: 4 tiles x 8 waves, 256: 2 tiles x 4
// waves, 512: 2 tiles x 2 waves): 64 x 16k keys at D = 64 76.0%, 64 x 8k at
// D = 256 83.2%, 64 x 4k at D = 512 79.2% of 8 TB/s, against 63-66% on the
// chunked kernel below.
constexpr int kDecSplitKeysMax = 2048;
constexpr int kDecSplitKeysMin = 512;
constexpr int kDecItemsPerWave = 2;
constexpr int kDecTileKeys = 16;
constexpr int kDecTilesInFlight = 2;

// ---- decode, pages of fewer than 1024 / 2D keys (fa_decode.hip): 32768
// elements (64 KB) of K per chunk, i.e. 32768 / D keys.  64 x 4k keys at
// D = 512 (16-key pages, before the streaming kernel took them): 63.8% of
// 8 TB/s; 64 x 16k keys at D = 128, pages of 1-8 keys: 65-67%.
constexpr int kDecChunkElems = 32768;

// ---- split-KV paged prefill (fa_fwd.hip paged_num_splits): no split when
// the query tiles alone give >= CU-count workgroups or the block table holds
// fewer than kSplitMinKeys keys; otherwise max(ceil(CUs / workgroups),
// ceil(keys / kSplitMaxRangeKeys)) ranges, but none shorter than
// kSplitMinRangeKeys and at most kMaxSplits.
// Evidence (2 sequences, 32 / 8 heads, D = 128, time per call in ms for
// 1 / 4 / 8 / 16 splits): 32k-key prefix + 128 tokens 0.955 / 0.277 / 0.171 /
// 0.192 (this rule: 8); 16k + 128: 0.487 / 0.153 / 0.104 / 0.128 (8);
// 32k + 512: 0.994 / 0.593 / 0.634 / 0.729 (5); 8k + 64: 0.252 / 0.087 /
// 0.062 / 0.080 (8).  The former rule (2 x CUs / workgroups ranges of at
// least 2048 keys) chose 16, 8, 4 and 4.
constexpr int kSplitMinKeys = 4096;
constexpr int kSplitMinRangeKeys = 1024;
constexpr int kSplitMaxRangeKeys = 8192;
constexpr int kMaxSplits = 64;

}  // namespace tiles
}  // namespace fa
