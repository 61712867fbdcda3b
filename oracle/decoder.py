"""CPU reference forward of the decoder the verification step runs (torch, fp32).

Restates the layer order of the HF Qwen3 text decoder layer the reference
verifies (transformers modeling_qwen3_vl.py Qwen3VLTextDecoderLayer /
Qwen3VLTextAttention / Qwen3VLTextMLP; respect/kernels/patch.py replaces its
linears and norms): pre-norm, q/k/v projections, q_norm / k_norm per head,
RoPE, GQA attention over the prompt and the allowed node slots, o
projection, residual add, post-attention norm, SwiGLU MLP, residual add;
final norm; fp32 vocabulary projection.  Activations are rounded to bf16 where
the model's bf16 tensors are (linear outputs, norms, residual sums, RoPE,
SwiGLU), attention is the exact softmax in float64.

Test infrastructure only: it checks the wiring of the GPU decoder (which
projection rows are q, k, v; where RoPE applies; which slots a row sees),
not bits -- bitwise parity of the GPU path is against its own 1-token path.
Pinned by: transformers' own Qwen3-VL text decoder on the CPU with the same
weights (logits within 3 % of the largest, where a RoPE sign, swapped k/v or
gate/up rows, dropped q/k norms, swapped layer norms or a row not seeing its
own slot each move them by 25 % or more); its pieces are oracle.norm (pinned
against PyTorch) and exact float64 attention; tests/test_oracle_decoder.py
also checks, on tiny models, that
its batched forward equals its own token-by-token forward, that the cache
slot layout does not matter, and that with a single visible key the q/k
weights cannot change the logits (the attention output is that key's value).
"""
from __future__ import annotations

import numpy as np
import torch

from . import norm as N


def _bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


def _lin(x, w):
    return _bf(x @ w.T)


class RefDecoder:
    """Holds float32 copies of a GPU ``Decoder``'s bf16 weights."""

    def __init__(self, model):
        c = model.cfg
        self.cfg = c
        f = lambda t: t.detach().float().cpu()
        self.embed = f(model.embed)
        self.layers = [dict(in_norm=f(l.in_norm), wqkv=f(l.wqkv), q_norm=f(l.q_norm), k_norm=f(l.k_norm),
                            wo=f(l.wo), post_norm=f(l.post_norm), wgu=f(l.wgu), wd=f(l.wd)) for l in model.layers]
        self.final_norm = f(model.final_norm)
        self.lm_head = f(model.lm_head)

    def _norm(self, x, w):
        return torch.from_numpy(N.rmsnorm(x.numpy(), w.numpy(), self.cfg.eps))

    def forward(self, ids, slots, positions, allow, kv=None):
        """ids [T]; token t writes cache slot slots[t] and rotates by positions[t];
        allow [T, S] bool: the cache slots row t attends to (its own included);
        kv: dict layer -> (K [HK, S, D], V) float32 holding earlier slots.
        Returns (fp32 logits [T, V], kv)."""
        c = self.cfg
        HQ, HK, D = c.heads, c.kv_heads, c.head_dim
        T = len(ids)
        S = allow.shape[1]
        cos, sin = N.rope_tables(np.asarray(positions), D, c.theta)
        cos, sin = torch.from_numpy(cos), torch.from_numpy(sin)
        x = self.embed[torch.as_tensor(ids)]
        if kv is None:
            kv = {}
        for li, L in enumerate(self.layers):
            y = self._norm(x, L["in_norm"])
            qkv = _lin(y, L["wqkv"])
            q = qkv[:, :HQ * D].reshape(T, HQ, D)
            k = qkv[:, HQ * D:(HQ + HK) * D].reshape(T, HK, D)
            v = qkv[:, (HQ + HK) * D:].reshape(T, HK, D)
            q = self._norm(q, L["q_norm"])
            k = self._norm(k, L["k_norm"])
            q = torch.from_numpy(N.rope(q.numpy(), cos.numpy()[:, None], sin.numpy()[:, None]))
            k = torch.from_numpy(N.rope(k.numpy(), cos.numpy()[:, None], sin.numpy()[:, None]))
            K, V = kv.get(li, (torch.zeros(HK, S, D), torch.zeros(HK, S, D)))
            for t, sl in enumerate(slots):
                K[:, int(sl)] = k[t]
                V[:, int(sl)] = v[t]
            kv[li] = (K, V)
            out = torch.empty(T, HQ, D)
            G = HQ // HK
            for h in range(HQ):
                s = (q[:, h].double() @ K[h // G].double().T) * D ** -0.5        # [T, S]
                s = s.masked_fill(~allow, float("-inf"))
                p = torch.softmax(s, dim=-1)
                out[:, h] = _bf((p @ V[h // G].double()).float())
            h_ = _lin(out.reshape(T, HQ * D), L["wo"])
            x = _bf(x + h_)
            y = self._norm(x, L["post_norm"])
            gu = _lin(y, L["wgu"])
            F = c.ffn
            m = torch.from_numpy(N.silu_mul(gu[:, :F].numpy(), gu[:, F:].numpy()))
            x = _bf(x + _lin(m, L["wd"]))
        y = self._norm(x, self.final_norm)
        return y @ self.lm_head.T, kv
