"""Benchmark of the MI355X attention path (one GPU).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--no-extra] [--no-cpu]
python bench.py --calibrate-copy      (256 MiB copies, for counter calibration)

Headline (`value`): BASELINE.json configs[1] — dense causal FlashAttention
forward + backward, fp16, q/k/v/dO [B=4, S=2048, H=16, D=128], one step =
tilelang_flash_attn_func forward + autograd backward over resident inputs.
value = algorithmic FLOPs per step / step time (FLOPs over unmasked pairs
only: fwd 4*D*H*pairs, bwd 2.5x fwd).

`roofline` covers the dominant launch of that step, the fa_bwd call (row
statistics, dK / dV storing the dS tiles, dQ from them), timed with HIP events
on the stream it is launched on; its `traffic` (HBM bytes per launch) comes from the counter
runs summarised in profiles/fa_bwd_c2_traffic.md.  `extra` reports the other
BASELINE configs and the north-star points (T1: S=8192 fwd+bwd, T2: decode
at 32k context) with their own roofline fractions; paged/decode reps flush
the 256 MB Infinity Cache.  Each entry's `ms` is GPU time per call (a spin
kernel ahead of the start event hides the Python wrapper), `api_ms` the
same interval without it, i.e. including host time the GPU spends idle.
`cpu_baseline` times the CPU oracle (fp32 PyTorch math, the reference math
path) on a bounded sample of the same workload on this host's cores.
After the headline's first warmup step (which carries the one-time kernel
load), ~0.3 s of fp16 matrix products bring the GPU clock out of its idle
state (clock_warmup); it is not a step and is not timed.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tilelang-fa-v100_amd"))
sys.path.insert(0, REPO)

import torch  # noqa: E402

PEAK_TFLOPS = 2516.6  # MI355X dense fp16/bf16 MFMA
PEAK_GBS = 8000.0     # MI355X HBM3E
METRIC = "attn TFLOP/s (prefill/bwd) + decode KV GB/s, % of MI355X roofline, 1 GPU"


# --------------------------------------------------------------------- workloads
# Seeded recipe: CPU generator per config, lengths first, then the page
# permutation, then q, k, v (then dO); N(0,1) in fp32 cast to the dtype.

def dense_inputs(B, S, H, D, dtype, device, seed=0, with_do=True):
    g = torch.Generator().manual_seed(seed)
    ts = [torch.randn(B, S, H, D, generator=g).to(dtype) for _ in range(4 if with_do else 3)]
    return [t.to(device) for t in ts]


def dense_pairs(sq, sk, causal):
    if not causal:
        return sq * sk
    off = sk - sq
    # sum_i clamp(i + off + 1, 0, sk)
    return sum(max(0, min(i + off + 1, sk)) for i in range(sq))


def paged_inputs(lens_q, lens_kv, prefixes, Hq, Hkv, D, dtype, device, g, page=16,
                 device_values=False):
    """Scattered-page cache (pool = sum of pages), block table padded with -1."""
    npg = [math.ceil(n / page) for n in lens_kv]
    pool = sum(npg)
    perm = torch.randperm(pool, generator=g)
    maxb = max(npg)
    bt = torch.full((len(lens_kv), maxb), -1, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(npg):
        bt[b, :n] = perm[cur:cur + n].to(torch.int32)
        cur += n
    T = sum(lens_q)
    if device_values:
        gd = torch.Generator(device=device).manual_seed(0)
        mk = lambda *s: torch.randn(*s, generator=gd, device=device, dtype=torch.float32).to(dtype)  # noqa: E731
        q = mk(T, Hq, D)
        kc = mk(pool, page, Hkv, D)
        vc = mk(pool, page, Hkv, D)
    else:
        q = torch.randn(T, Hq, D, generator=g).to(dtype).to(device)
        kc = torch.randn(pool, page, Hkv, D, generator=g).to(dtype).to(device)
        vc = torch.randn(pool, page, Hkv, D, generator=g).to(dtype).to(device)
    qsl = torch.tensor([0] + torch.tensor(lens_q).cumsum(0).tolist(), dtype=torch.int32)
    return dict(q=q, k_cache=kc, v_cache=vc, block_table=bt.to(device),
                seq_lens=torch.tensor(lens_kv, dtype=torch.int32, device=device),
                query_start_loc=qsl.to(device),
                prefix_kv_lens=torch.tensor(prefixes, dtype=torch.int32, device=device))


def c3_lens():
    g = torch.Generator().manual_seed(0)
    return torch.randint(512, 4097, (8,), generator=g).tolist(), g


def c4_lens():
    g = torch.Generator().manual_seed(0)
    return torch.randint(1024, 32769, (64,), generator=g).tolist(), g


def c5_prefix():
    g = torch.Generator().manual_seed(0)
    return torch.randint(0, 8193, (16,), generator=g).tolist(), g


def decode_bytes(lens, Hq, Hkv, D, page=16, elem=2):
    kv = sum(lens) * Hkv * D * 2 * elem
    qo = len(lens) * Hq * D * elem * 2
    bt = sum(math.ceil(n / page) for n in lens) * 4 + 4 * len(lens)
    return kv + qo + bt


# --------------------------------------------------------------------- timing

class CacheFlush:
    """Reads a 512 MB buffer so the 256 MB Infinity Cache holds no inputs.

    A read, not a fill: a fill leaves the cache full of dirty lines whose
    write-back then lands inside the next timed call (measured: C4 decode
    0.719 ms after a fill, 0.681 ms after a read of the same buffer).
    """

    def __init__(self, device):
        self.buf = torch.ones(128 << 20, dtype=torch.int32, device=device)

    def __call__(self):
        self.buf.sum()


_SLEEP_CYCLES = None


def _sleep_cycles(target_ms=1.0):
    """Argument of torch.cuda._sleep that keeps the GPU busy for ~target_ms."""
    global _SLEEP_CYCLES
    if _SLEEP_CYCLES is None:
        n = 1 << 20
        torch.cuda._sleep(n)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        torch.cuda._sleep(n)
        e.record()
        e.synchronize()
        _SLEEP_CYCLES = max(1, int(n * target_ms / max(s.elapsed_time(e), 1e-3)))
    return _SLEEP_CYCLES


def time_reps(fn, reps, warmup, flush=None):
    """Median per-call times (ms): (gpu, api).

    gpu: a spin kernel queued ahead of the start event keeps the GPU busy
    while Python prepares the call, so the interval holds only the GPU work
    the call enqueues.  api: the same without the spin kernel, so host time
    during which the GPU idles is included (the cost a caller sees).
    """
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    out = []
    for hide_host in (True, False):
        times = []
        for _ in range(reps):
            if flush is not None:
                flush()
            if hide_host:
                torch.cuda._sleep(_sleep_cycles())
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            e.synchronize()
            times.append(s.elapsed_time(e))
        out.append(statistics.median(times))
    return out[0], out[1]


def flop_entry(name, flops, ms, api_ms=None, extra=None):
    tf = flops / (ms * 1e-3) / 1e12
    d = {"ms": round(ms, 4), "gflop": round(flops / 1e9, 2), "tflops": round(tf, 1),
         "frac_of_peak": round(tf / PEAK_TFLOPS, 4)}
    if api_ms is not None:
        d["api_ms"] = round(api_ms, 4)
    if extra:
        d.update(extra)
    return name, d


def bytes_entry(name, nbytes, ms, api_ms=None, extra=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    d = {"ms": round(ms, 4), "gbytes": round(nbytes / 1e9, 3), "gbs": round(gbs, 1),
         "frac_of_peak": round(gbs / PEAK_GBS, 4)}
    if api_ms is not None:
        d["api_ms"] = round(api_ms, 4)
        d["api_gbs"] = round(nbytes / (api_ms * 1e-3) / 1e9, 1)
    if extra:
        d.update(extra)
    return name, d


def profiled_traffic(name):
    """HBM bytes per launch recorded by the counter runs in profiles/<name>_traffic.md.

    The summary holds a line `traffic_bytes_per_launch: N` (FETCH_SIZE and
    WRITE_SIZE per dispatch, scaled by the copy-kernel calibration it
    states).  None when no summary has been recorded.
    """
    path = os.path.join(REPO, "profiles", f"{name}_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def device_info(device):
    """The box's own matrix rate next to the attention numbers.

    Boxes of this pool run the same kernels up to ~13% apart in the
    matrix-bound points (decode, HBM-bound, matches to ~1%): the shader clock
    under sustained matrix load differs.  An fp16 8192^3 matrix product
    through torch (hipBLASLt) is timed after the headline, so a reader can
    tell a slow box from a slow kernel.
    """
    props = torch.cuda.get_device_properties(device)
    a = torch.randn(8192, 8192, device=device, dtype=torch.float16)
    b = torch.randn(8192, 8192, device=device, dtype=torch.float16)
    for _ in range(3):
        a @ b
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(10):
        a @ b
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / 10
    return {"name": props.name, "arch": getattr(props, "gcnArchName", "?"),
            "compute_units": props.multi_processor_count,
            "fp16_gemm_8192_tflops": round(2 * 8192 ** 3 / (ms * 1e-3) / 1e12, 1)}


def clock_warmup(device, seconds=0.3):
    """Keeps the GPU busy with fp16 matrix products for `seconds`.

    The MI355X clock ramps up over ~0.3 s of continuous load after the GPU
    idles (here: while inputs are drawn and kernels load on the host).
    Measured on C2 in a fresh process, per 5-step group: 0.41-0.42 ms/step
    for the first 20 steps, reaching 0.387 only after ~40 steps; with this
    warm-up after the first step, 0.388-0.389 from the second step on.  0.1 s
    was not enough.  It is not an attention step and is outside the timed
    region.
    """
    a = torch.randn(4096, 4096, device=device, dtype=torch.float16)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            a @ a
        torch.cuda.synchronize()


# --------------------------------------------------------------------- legs

def headline(fa, steps, warmup, dev):
    B, S, H, D = 4, 2048, 16, 128
    q, k, v, do = dense_inputs(B, S, H, D, torch.float16, dev)
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()
    pairs = dense_pairs(S, S, True)
    f_fwd = 4 * D * H * pairs * B
    f_step = 3.5 * f_fwd

    def step():
        q.grad = k.grad = v.grad = None  # fresh gradients: the step is fwd + bwd only
        out = fa.tilelang_flash_attn_func(q, k, v, causal=True)
        out.backward(do)

    # The first step pays the one-time library and kernel load (~30 ms of host
    # work with the GPU idle), so the clock warm-up follows it.
    if warmup > 0:
        step()
        torch.cuda.synchronize()
    clock_warmup(dev)
    for _ in range(warmup - 1):
        step()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        step()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps

    # Dominant launch: fa_bwd (pre + main + dQ convert) through the C ABI.
    from tilelang_fa_v100 import _dense, _lib
    qd, kd, vd = q.detach(), k.detach(), v.detach()
    out, lse = _dense.forward(qd, kd, vd, D ** -0.5, True)
    dq, dk, dv = (torch.empty_like(t) for t in (qd, kd, vd))
    a = _dense.bwd_args(qd, kd, vd, out, do, lse, dq, dk, dv, D ** -0.5, True, False)
    lib = _lib.load()
    nbytes = lib.fa_bwd_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(qd.device)

    def bwd():
        _lib.check(lib.fa_bwd(ctypes.byref(a), ws.data_ptr(), nbytes, stream), "fa_bwd")

    bwd_ms, bwd_api = time_reps(bwd, max(steps, 20), 3)
    fwd_ms, fwd_api = time_reps(lambda: _dense.forward(qd, kd, vd, D ** -0.5, True),
                                max(steps, 20), 3)
    bwd_tf = 2.5 * f_fwd / (bwd_ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "achieved": round(bwd_tf, 1), "peak": PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(bwd_tf / PEAK_TFLOPS, 4),
                "traffic": profiled_traffic("fa_bwd_c2"),
                "kernel": "fa_bwd (bwd_stats row statistics, bwd_main_mfma dK/dV + dS tiles, "
                          "bwd_dq_ds dQ)",
                "launch_ms": round(bwd_ms, 4), "algorithmic_gflop": round(2.5 * f_fwd / 1e9, 2)}
    parts = dict([flop_entry("C2_fwd", f_fwd, fwd_ms, fwd_api),
                  flop_entry("C2_bwd", 2.5 * f_fwd, bwd_ms, bwd_api)])
    return ms, f_step, roofline, parts


def extras(fa, dev, reps):
    res = {}
    flush = CacheFlush(dev)
    # C1: dense non-causal forward fp16 [1,512,16,64]
    q, k, v = dense_inputs(1, 512, 16, 64, torch.float16, dev, with_do=False)
    ms, api = time_reps(lambda: fa.tilelang_flash_attn_func(q, k, v), reps, 5)
    res.update([flop_entry("C1_fwd", 4 * 64 * 16 * 512 * 512, ms, api)])

    # T1: dense causal fwd+bwd S=8192 D=128, B=2 H=16
    q, k, v, do = dense_inputs(2, 8192, 16, 128, torch.float16, dev)
    for t in (q, k, v):
        t.requires_grad_()
    f_fwd = 4 * 128 * 16 * dense_pairs(8192, 8192, True) * 2

    def t1():
        q.grad = k.grad = v.grad = None
        o = fa.tilelang_flash_attn_func(q, k, v, causal=True)
        o.backward(do)

    ms, api = time_reps(t1, max(reps // 2, 5), 2)
    res.update([flop_entry("T1_fwd_bwd", 3.5 * f_fwd, ms, api)])
    ms, api = time_reps(lambda: fa.tilelang_flash_attn_func(q.detach(), k.detach(), v.detach(),
                                                          causal=True), reps, 3)
    res.update([flop_entry("T1_fwd", f_fwd, ms, api)])
    del q, k, v, do

    # head_dim 256 at the T1 sequence length (B=2, H=8: the same bytes per row)
    q, k, v, do = dense_inputs(2, 8192, 8, 256, torch.float16, dev)
    for t in (q, k, v):
        t.requires_grad_()
    f_fwd = 4 * 256 * 8 * dense_pairs(8192, 8192, True) * 2

    def t1_d256():
        q.grad = k.grad = v.grad = None
        o = fa.tilelang_flash_attn_func(q, k, v, causal=True)
        o.backward(do)

    ms, api = time_reps(t1_d256, max(reps // 4, 3), 1)
    res.update([flop_entry("T1_D256_fwd_bwd", 3.5 * f_fwd, ms, api)])
    ms, api = time_reps(lambda: fa.tilelang_flash_attn_func(q.detach(), k.detach(), v.detach(),
                                                          causal=True), reps, 3)
    res.update([flop_entry("T1_D256_fwd", f_fwd, ms, api)])
    del q, k, v, do

    # C3: paged causal prefill fp16, 8 seqs U[512,4096], 32/8 heads, D=128
    lens, g = c3_lens()
    c = paged_inputs(lens, lens, [0] * 8, 32, 8, 128, torch.float16, dev, g)
    pairs = sum(n * (n + 1) // 2 for n in lens)
    run = lambda: fa.tilelang_paged_forward(**c)  # noqa: E731
    ms, api = time_reps(run, reps, 3, flush)
    res.update([flop_entry("C3_paged_prefill", 4 * 128 * 32 * pairs, ms, api)])
    del c

    # C5: chunked prefill with prefix, bf16, 16 x 512 new tokens, 64/8 heads
    pf, g = c5_prefix()
    c = paged_inputs([512] * 16, [p + 512 for p in pf], pf, 64, 8, 128, torch.bfloat16, dev, g)
    pairs = sum(sum(min(p + t + 1, p + 512) for t in range(512)) for p in pf)
    run = lambda: fa.tilelang_paged_forward(**c)  # noqa: E731
    ms, api = time_reps(run, reps, 3, flush)
    res.update([flop_entry("C5_chunked_prefill_bf16", 4 * 128 * 64 * pairs, ms, api)])
    del c

    # P1: long-prefix prefill (split-KV): 2 sequences x 128 new tokens after a
    # 32k-key prefix, 32/8 heads, D=128, fp16.  Unsplit, the query tiles
    # give 32 workgroups (2 x 4 row tiles x 8 KV heads); the library splits
    # the keys.
    from tilelang_fa_v100._paged_adapter import paged_forward_splits
    pf = [32768, 32768]
    g = torch.Generator().manual_seed(0)
    c = paged_inputs([128] * 2, [p + 128 for p in pf], pf, 32, 8, 128, torch.float16, dev, g,
                     device_values=True)
    pairs = sum(sum(p + t + 1 for t in range(128)) for p in pf)
    ms, api = time_reps(lambda: fa.tilelang_paged_forward(**c), reps, 3, flush)
    ms1, api1 = time_reps(lambda: paged_forward_splits(**c, num_splits=1), reps, 3, flush)
    res.update([flop_entry("P1_long_prefix_prefill_split", 4 * 128 * 32 * pairs, ms, api,
                           extra={"unsplit_ms": round(ms1, 4),
                                  "unsplit_tflops": round(4 * 128 * 32 * pairs / ms1 / 1e9, 1)})])
    del c

    # C4 / T2: paged decode, batch 64, 32/8 heads, D=128
    for name, lens_fn in (("C4_decode", lambda: c4_lens()),
                          ("T2_decode_32k", lambda: ([32768] * 64, torch.Generator().manual_seed(0)))):
        lens, g = lens_fn()
        c = paged_inputs([1] * 64, lens, [0] * 64, 32, 8, 128, torch.float16, dev, g,
                         device_values=True)
        qd = c["q"].view(64, 32, 128)
        run = lambda: fa.tilelang_decode_forward(qd, c["k_cache"], c["v_cache"],  # noqa: E731
                                                 c["block_table"], c["seq_lens"])
        ms, api = time_reps(run, reps, 3, flush)
        res.update([bytes_entry(name, decode_bytes(lens, 32, 8, 128), ms, api)])
        del c, qd

    # Decode at the other head dims (64 sequences, 32 / 8 heads, fp16).
    for name, D, n in (("decode_D64_64x16k", 64, 16384), ("decode_D256_64x8k", 256, 8192),
                       ("decode_D512_64x4k", 512, 4096)):
        lens = [n] * 64
        c = paged_inputs([1] * 64, lens, [0] * 64, 32, 8, D, torch.float16, dev,
                         torch.Generator().manual_seed(0), device_values=True)
        qd = c["q"].view(64, 32, D)
        run = lambda: fa.tilelang_decode_forward(qd, c["k_cache"], c["v_cache"],  # noqa: E731
                                                 c["block_table"], c["seq_lens"])
        ms, api = time_reps(run, reps, 3, flush)
        res.update([bytes_entry(name, decode_bytes(lens, 32, 8, D), ms, api)])
        del c, qd
    return res


def cpu_model() -> str:
    """The host CPU's model name (lscpu / /proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s=10.0):
    """Oracle fp32 fwd+bwd over C2's own (batch, head) slices.

    C2's inputs are drawn with the headline's recipe (seed 0, [4, 2048, 16,
    128] fp16) and the oracle runs one (b, h) slice at a time, in order;
    whole passes over all 64 slices repeat until budget_s has elapsed (a
    pass takes ~2 s on 8-16 cores), and the rate is taken over all of them.
    """
    from oracle import attention_ref as ref
    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    B, S, H, D = 4, 2048, 16, 128
    q, k, v, do = dense_inputs(B, S, H, D, torch.float16, "cpu")
    per_head = 3.5 * 4 * D * dense_pairs(S, S, True)
    sl = lambda t, b, h: t[b:b + 1, :, h:h + 1]  # noqa: E731
    ref.dense_attention(sl(q, 0, 0), sl(k, 0, 0), sl(v, 0, 0), causal=True)  # warm-up
    done, passes, t0 = 0, 0, time.perf_counter()
    while passes == 0 or time.perf_counter() - t0 < budget_s:
        for bh in range(B * H):
            b, h = divmod(bh, H)
            ref.dense_attention(sl(q, b, h), sl(k, b, h), sl(v, b, h), causal=True)
            ref.dense_attention_backward(sl(q, b, h), sl(k, b, h), sl(v, b, h),
                                         sl(do, b, h), causal=True)
            done += 1
        passes += 1
    el = time.perf_counter() - t0
    tf = done * per_head / el / 1e12
    return {"value": round(tf, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "cpu_model": cpu_model(), "kind": "port",
            "sample": f"C2 fwd+bwd, all {B * H} (batch, head) slices of the C2 inputs (seed 0) "
                      f"x {passes} passes, fp32 oracle (oracle/attention_ref.py) on CPU, "
                      f"{el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # ~40 ms of untimed steps before timing: with 5 the GPU's clocks and caches had not
    # settled (0.424 ms/step for 20 steps vs 0.389 ms/step after 50 warmup steps).
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 5 device copies of 256 MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        # A plain copy of known size: FETCH_SIZE / WRITE_SIZE per dispatch of
        # this kernel against 256 MiB give the counters' scale factors.
        x = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": 256 << 20, "dispatches": 5}), flush=True)
        return
    import tilelang_fa_v100 as fa
    print(f"[bench] headline C2: warmup {args.warmup}, steps {args.steps}", file=sys.stderr, flush=True)
    ms, f_step, roof, parts = headline(fa, args.steps, args.warmup, dev)
    extra = dict(parts)
    if not args.no_extra:
        print("[bench] extra configs", file=sys.stderr, flush=True)
        extra.update(extras(fa, dev, args.reps))
    device = device_info(dev)
    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline()
    line = {
        "metric": METRIC,
        "value": round(f_step / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "C2: dense causal FA fwd+bwd, fp16, q/k/v/dO [4,2048,16,128], "
                               "seed 0, scale 1/sqrt(128)",
                   "global_batch": 4, "seq_len": 2048, "heads": 16, "head_dim": 128,
                   "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "device": device,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
