"""Public API: drop-in for tilelang_fa_v100/interface.py of the reference.

Same four functions, same signatures and defaults, same return conventions:
  tilelang_flash_attn_func / tilelang_flash_attn_gpu   (interface.py:59-80,101)
  tilelang_paged_forward                                (interface.py:83-98)
  tilelang_decode_forward                               (interface.py:104-117)
and the autograd Function FlashAttnTileLangVFunc (interface.py:12-56).

Behavioural notes relative to the reference (each one only removes a
limitation):
  * softmax_scale is honoured by every kernel (the reference's dense and
    decode kernels always use 1/sqrt(D); identical at the default);
  * fp16 and bf16 are accepted; the output dtype is q's dtype;
  * dense K/V may have fewer heads than Q (GQA, contiguous head groups);
  * a query row that sees no key gets out = 0 and lse = -inf (the reference
    produces NaN);
  * window_size is honoured with FlashAttention-2 semantics (key j visible to
    query i iff i + off - left <= j <= i + off + right, off = Sk - Sq, -1 =
    unbounded, causal implies right = 0); the reference parses it and then
    ignores it (:33).  The default (-1, -1) is identical.
"""
from __future__ import annotations

import torch

from . import _dense
from ._checks import require_cuda, require_half, require_same
from ._decode_adapter import decode_forward as _decode_forward
from ._paged_adapter import paged_forward as _paged_forward


class FlashAttnTileLangVFunc(torch.autograd.Function):
    """Autograd Function for dense FlashAttention (interface.py:12-56)."""

    @staticmethod
    def forward(ctx, q, k, v, dropout_p, softmax_scale, causal, window_size,
                softcap, alibi_slopes, deterministic, return_softmax):
        if dropout_p != 0.0:
            raise NotImplementedError("dropout not supported")
        if alibi_slopes is not None:
            raise NotImplementedError("alibi not supported")
        if softcap != 0.0:
            raise NotImplementedError("softcap not supported")
        for name, t in (("q", q), ("k", k), ("v", v)):
            require_half(t, name)
        require_same({"q": q, "k": k, "v": v}, "dtype")
        shapes = _dense.check_shapes(q, k, v)
        for name, t in (("q", q), ("k", k), ("v", v)):
            require_cuda(t, name)
        require_same({"q": q, "k": k, "v": v}, "device")
        scale = softmax_scale if softmax_scale is not None else q.shape[-1] ** -0.5
        window = _dense.window_bounds(window_size)
        # Without gradients and without a requested LSE (inference) the kernel
        # skips the LSE store, as the reference's tilelang_forward does
        # (_kernels_forward.py:176-185).
        with_lse = bool(return_softmax) or any(ctx.needs_input_grad[:3])
        out, lse = _dense.forward(q, k, v, scale, causal, window, shapes=shapes,
                                  with_lse=with_lse)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal = bool(causal)
        ctx.window = window
        ctx.softmax_scale = float(scale)
        ctx.deterministic = bool(deterministic)
        if return_softmax:
            return out, lse, None
        return out

    @staticmethod
    def backward(ctx, dout, *args):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = _dense.backward(q, k, v, out, dout, lse, ctx.softmax_scale,
                                     ctx.causal, ctx.deterministic, ctx.window)
        return dq, dk, dv, None, None, None, None, None, None, None, None


def tilelang_flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None,
                             causal=False, window_size=(-1, -1), softcap=0.0,
                             alibi_slopes=None, deterministic=False,
                             return_attn_probs=False):
    """FA2-compatible flash attention.

    Args:
        q: [B, Sq, H, D]; k, v: [B, Sk, Hk, D] with H % Hk == 0.
        causal: bottom-right aligned causal mask (key j visible to query i
            iff j <= i + Sk - Sq).
        window_size: (left, right) sliding window, -1 = unbounded.
        softmax_scale: default 1/sqrt(D).
        return_attn_probs: return (out, lse [B, H, Sq] fp32, None).
    Returns:
        out [B, Sq, H, D] in q's dtype, or (out, lse, None).
    """
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    return FlashAttnTileLangVFunc.apply(
        q, k, v, dropout_p, softmax_scale, causal,
        window_size, softcap, alibi_slopes, deterministic, return_attn_probs,
    )


def tilelang_paged_forward(q, k_cache, v_cache, block_table, seq_lens,
                           query_start_loc, prefix_kv_lens, out=None,
                           block_size=16, num_kv_heads=None,
                           softmax_scale=None, causal=True,
                           sliding_window_q=-1, sliding_window_k=-1):
    """Paged FlashAttention forward for vLLM: returns (out, softmax_lse)."""
    return _paged_forward(
        q, k_cache, v_cache, block_table, seq_lens,
        query_start_loc, prefix_kv_lens, out=out,
        block_size=block_size, num_kv_heads=num_kv_heads,
        softmax_scale=softmax_scale, causal=causal,
        sliding_window_q=sliding_window_q, sliding_window_k=sliding_window_k,
    )


tilelang_flash_attn_gpu = tilelang_flash_attn_func


def tilelang_decode_forward(q, k_cache, v_cache, block_table, seq_lens,
                            block_size=16, num_kv_heads=None,
                            softmax_scale=None):
    """Paged decode forward for vLLM: q [B, Hq, D] -> output [B, Hq, D]."""
    return _decode_forward(
        q, k_cache, v_cache, block_table, seq_lens,
        block_size=block_size, num_kv_heads=num_kv_heads,
        softmax_scale=softmax_scale,
    )
