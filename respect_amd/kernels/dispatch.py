"""Route the target model's SDPA attention to the trie-verification kernel.

Same module interface as respect/kernels/dispatch.py:18-140: ``install(PL)``,
``uninstall()``, ``STATE``, ``STATS``, ``BM``, ``MSTEP``, ``MMAX``, ``NSTEP``,
``NMAX``, ``BNB``, ``CFG`` and ``unified_forward`` with the signature of
transformers' SDPA attention function.  The key axis is split at the prompt
length PL: slots before PL are the prompt segment (never masked), slots from PL
on the node segment, masked by the caller's 4-D mask or, without one, causally.
Calls that do not fit (batch > 1, dropout, attention weights requested, sizes
beyond the limits, a prompt column that the mask closes, shapes the kernel does
not build) fall back to the original SDPA function, as the reference does.

What differs from the reference is only what the HIP kernel makes unneeded:
its arithmetic does not depend on the number of query rows or node slots, so
nothing is padded to MSTEP / NSTEP; q, the node K/V and the mask are passed as
views of the caller's tensors (no zero-fill and copy); and the kernel writes
the output directly in the [1, q, H, D] layout the caller returns.  MSTEP,
NSTEP and BNB are kept as module attributes with the reference's values.
"""
from __future__ import annotations

import torch
import transformers.integrations.sdpa_attention as SA

from .attention import trie_attn

ORIG = SA.sdpa_attention_forward
BM = 64
MSTEP = 64
MMAX = 1024
NSTEP = 32
NMAX = 4096
BNB = 16
STATE = {"PL": None}
CFG = dict(BM=BM, BN=128, num_warps=4, num_stages=1)
STATS = {"kernel": 0, "fallback": 0}
_PROMPT_OK: dict = {}


def _fb(module, query, key, value, attention_mask, dropout, scaling, is_causal, kwargs):
    STATS["fallback"] += 1
    return ORIG(module, query, key, value, attention_mask, dropout, scaling, is_causal, **kwargs)


def _allow_from(am):
    a = am[0, 0] if am.dim() == 4 else am
    return a if a.dtype == torch.bool else (a == 0)


def _prompt_all_open(allow, PL, key):
    """Whether every query row may attend to every prompt slot (one host sync per mask)."""
    v = _PROMPT_OK.get(key)
    if v is None:
        v = bool(allow[:, :PL].all())
        if len(_PROMPT_OK) >= 8:
            _PROMPT_OK.clear()
        _PROMPT_OK[key] = v
    return v


def unified_forward(module, query, key, value, attention_mask, dropout=0.0, scaling=None, is_causal=None,
                    **kwargs):
    """query [1, H, q, D], key/value [1, HK, PL + n, D] -> ([1, q, H, D], None)."""
    args = (module, query, key, value, attention_mask, dropout, scaling, is_causal, kwargs)
    PL = STATE["PL"]
    if PL is None or query.shape[0] != 1 or dropout != 0.0 or kwargs.get("output_attentions", False):
        return _fb(*args)
    q_len, n_kv = query.shape[2], key.shape[2]
    n_node = n_kv - PL
    if n_node < q_len or n_node < 0 or q_len > MMAX or n_node > NMAX:
        return _fb(*args)
    H, D = query.shape[1], query.shape[3]
    dev = query.device

    if attention_mask is not None and attention_mask.dim() == 4:
        if attention_mask.shape[-1] != n_kv or attention_mask.shape[-2] != q_len:
            return _fb(*args)
        allow = _allow_from(attention_mask)
        if not _prompt_all_open(allow, PL, (attention_mask.data_ptr(), tuple(attention_mask.shape))):
            return _fb(*args)
        msk = allow[:, PL:]
    else:
        # causal over the node segment: query i sits at node slot n_node - q_len + i
        first = n_node - q_len
        rows = torch.arange(q_len, device=dev)[:, None] + first
        msk = torch.arange(n_node, device=dev)[None, :] <= rows

    scale = scaling if scaling is not None else D ** -0.5
    y = torch.empty((1, q_len, H, D), dtype=query.dtype, device=dev)
    try:
        trie_attn(query[0], key[0][:, :PL], value[0][:, :PL], key[0][:, PL:], value[0][:, PL:], msk, scale,
                  out=y[0].transpose(0, 1))
    except Exception:
        return _fb(*args)
    STATS["kernel"] += 1
    return y, None


def install(PL):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    STATE["PL"] = PL
    _PROMPT_OK.clear()
    SA.sdpa_attention_forward = unified_forward
    ALL_ATTENTION_FUNCTIONS["sdpa"] = unified_forward


def uninstall():
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    STATE["PL"] = None
    _PROMPT_OK.clear()
    SA.sdpa_attention_forward = ORIG
    ALL_ATTENTION_FUNCTIONS["sdpa"] = ORIG
