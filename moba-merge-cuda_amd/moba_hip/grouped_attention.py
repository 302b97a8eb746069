"""MoBA GQA/MQA/MHA prefill entry (`opt_hip`) on the gfx950 HIP kernels.

Drop-in for ``opt_gqa_cuda`` (src/moba_opt/grouped_attention.py:29-99):
same signature ``(q [T,Hq,D], k/v [T,Hkv,D], cu_seqlens int32 [B+1],
max_seqlen, config)``, same config keys (``chunk_size``, ``topk``,
``causal``, ``dropout``, ``route_precision`` in {'upstream','fp32'},
``deterministic_merge``, ``stable_routes``), same ValueErrors, a
differentiable output in the input dtype, and the same ``ROUTE_HOOK`` test
hook called with ``cu_chunk``, ``filtered_chunk_indices``, ``chunk_to_batch`` and
``selected [F,Hq,T] bool``.

Differences that are properties of this implementation, not options:
  * routing is always the canonical deterministic rule (fixed fp32 summation
    order, exact ties -> lowest chunk), so ``stable_routes`` only documents it;
  * the merge is always deterministic (fixed ascending-chunk order, no atomics),
    so ``deterministic_merge`` only documents it;
  * no packed copies of q / k / v are made: kernels gather rows in place.
"""
import torch

from .api import register
from .baseline_adapter import _validate
from .ops import prefill as P

ROUTE_HOOK = None  # test-only; None in all performance paths

_PRECISION = {"upstream": 0, "fp32": 1}


def _selected_mask(plan, rt, T, hq, device):
    """[F,Hq,T] bool view of the slot lists (for ROUTE_HOOK only)."""
    sel = rt.sel.long()
    valid = sel >= 0
    batch = plan.dev("chunk_batch").long()
    f = sel.clamp_min(0) - batch[sel.clamp_min(0)]
    s_idx = torch.arange(T, device=device).view(T, 1, 1).expand_as(sel)
    h_idx = torch.arange(hq, device=device).view(1, hq, 1).expand_as(sel)
    mask = torch.zeros((plan.num_filtered, hq, T), dtype=torch.bool, device=device)
    mask[f[valid], h_idx[valid], s_idx[valid]] = True
    return mask


class MobaHipAttention(torch.autograd.Function):
    """Forward: route -> pack -> sparse attention + merge; backward with the
    global O/LSE (mixed_attention.py:141-225 semantics)."""

    @staticmethod
    def forward(ctx, q, k, v, plan, precision):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        rt = None
        if not plan.fallback:
            rt = P.route(plan, q, k, precision)
            if ROUTE_HOOK is not None:
                dev = q.device
                ROUTE_HOOK(cu_chunk=plan.dev("cu_chunk"),
                           filtered_chunk_indices=plan.dev("filtered")[:plan.num_filtered].long(),
                           chunk_to_batch=plan.dev("chunk_batch"),
                           selected=_selected_mask(plan, rt, q.shape[0], q.shape[1], dev))
        out, lse = P.forward(plan, q, k, v, rt)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.plan, ctx.rt = plan, rt
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = P.backward(ctx.plan, q, k, v, out, lse, dout.contiguous(), ctx.rt)
        return dq, dk, dv, None, None


def _config_flags(config):
    precision = config.get("route_precision", "upstream")
    deterministic = config.get("deterministic_merge", False)
    stable = config.get("stable_routes", False)
    if precision not in _PRECISION:
        raise ValueError("route_precision")
    if not isinstance(deterministic, bool) or not isinstance(stable, bool):
        raise ValueError("routing flags must be bool")
    return _PRECISION[precision]


def moba_hip_attention(q, k, v, cu_seqlens, max_seqlen, config, *, allow_gqa=True,
                       return_lse=False):
    cu = _validate(q, k, v, cu_seqlens, allow_gqa=allow_gqa, max_seqlen=max_seqlen,
                   config=config)
    precision = _config_flags(config)
    plan = P.get_plan(cu, int(config["chunk_size"]), q.shape[1], k.shape[1], q.shape[2],
                      int(config["topk"]), q.device)
    out, lse = MobaHipAttention.apply(q, k, v, plan, precision)
    return (out, lse) if return_lse else out


def opt_hip(q, k, v, cu_seqlens, max_seqlen, config):
    """GQA/MQA/MHA MoBA prefill (registry name ``opt_hip``)."""
    return moba_hip_attention(q, k, v, cu_seqlens, max_seqlen, config)


def opt_hip_mha(q, k, v, cu_seqlens, max_seqlen, config):
    """MHA-only entry with the MHA contract of moba_attn_varlen_opt
    (mixed_attention.py:228-420); registry name ``opt_merge_hip``."""
    return moba_hip_attention(q, k, v, cu_seqlens, max_seqlen, config, allow_gqa=False)


register("opt_hip", opt_hip)
register("opt_merge_hip", opt_hip_mha)
