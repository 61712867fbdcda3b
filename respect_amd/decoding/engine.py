"""Decoder forward of the verification step, on the C-ABI kernels only.

A Qwen3-style dense GQA decoder (the text model the reference verifies with:
pre-norm layers, q_norm / k_norm, RoPE, SwiGLU MLP, untied vocabulary head)
with random-initialised weights -- there is no network to fetch checkpoints.
Every arithmetic step goes through librespect_amd:

    x = embed[ids]                                   (row gather)
    y = rmsnorm(x)                                   rspx_rmsnorm
    per layer:
      qkv = y . Wqkv^T                               rspx_linear_partials
      q, cache[k, v] at the tokens' slots            rspx_qkv_rope_cache_partials
      a = attention(q; prompt K/V, node K/V, mask)   rspx_trie_attn
      h = a . Wo^T                                   rspx_linear_partials
      x, y = x + h, rmsnorm(x + h)                   rspx_add_rmsnorm_partials
      g|u = y . Wgu^T ; m = silu(g) * u              rspx_linear_silu (or rspx_linear, rspx_silu_mul)
      h = m . Wd^T ; x, y = x + h, rmsnorm(x + h)    rspx_linear_partials, rspx_add_rmsnorm_partials

A projection feeding an epilogue is left as its fp32 K-chunk partials and
the epilogue adds them in chunk order and rounds to bf16 -- the exact value
rspx_linear would store -- so no separate reduction launch is needed.
    logits = y . Wlm^T (fp32)                        rspx_linear

The normalised rows y, the attention output and the SwiGLU output m, read
only by linear layers, stay in the tiled activation layout (RSPX_TILED), and
every weight matrix is held in the tiled weight layout
(kernels.gemm.tile_weight): the linear layers then load both operands a whole
MFMA tile per instruction, with the same result bits as from row-major
operands.

Each kernel computes a row with arithmetic that does not depend on how many
rows the call carries, and attention folds a row's node slots in slot order,
so a token verified inside a trie gets the same logits and KV bits as when it
is decoded alone -- the property the reference's verification relies on
(respect/decoding/verify.py:12-46, respect/decoding/sequential.py:17-42).
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch

from .. import _lib
from ..kernels.attention import raise_if_gave_up, status_word, trie_attn
from ..kernels.gemm import TiledWeight, tile_weight
from ..system.fused import rope_tables
from .acceptance import greedy_token


@dataclass(frozen=True)
class DecoderConfig:
    layers: int = 36
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 12288
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1.0e6

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def weight_bytes(self) -> int:
        """bf16 bytes of every weight one forward reads (embedding rows aside)."""
        H, F, V = self.hidden, self.ffn, self.vocab
        per_layer = self.qkv_rows * H + H * self.heads * self.head_dim + 2 * F * H + H * F + 2 * H + 2 * self.head_dim
        return 2 * (self.layers * per_layer + V * H + H)


class Layer:
    """One decoder layer.  The projections are held tiled (``t*``, what the
    kernels read); ``wqkv``, ``wo``, ``wgu`` and ``wd`` give them back as
    row-major [N, K] copies for references and tests."""

    def __init__(self, cfg: DecoderConfig, g: torch.Generator, device, std: float):
        H, D, F = cfg.hidden, cfg.head_dim, cfg.ffn

        def w(*shape):
            return (torch.randn(*shape, generator=g, device=device) * std).to(torch.bfloat16)

        def norm_w(n):
            return (1.0 + torch.randn(n, generator=g, device=device) * std).to(torch.bfloat16)

        self.in_norm = norm_w(H)
        self.tqkv = tile_weight(w(cfg.qkv_rows, H))  # [q | k | v] rows
        self.q_norm = norm_w(D)
        self.k_norm = norm_w(D)
        self.tout = tile_weight(w(H, cfg.heads * D))
        self.post_norm = norm_w(H)
        wgu = w(2 * F, H)                            # [gate | up] rows
        self.tdown = tile_weight(w(H, F))
        # With one K chunk the gate/up product carries SwiGLU in its epilogue
        # (rspx_linear_silu), which wants the rows interleaved: 2i gate i, 2i + 1 up i.
        self.gu_fused = _lib.lib().rspx_linear_splits(2 * F, H) == 1
        self.tgu = tile_weight(wgu.view(2, F, H).transpose(0, 1).reshape(2 * F, H) if self.gu_fused else wgu)

    @property
    def wqkv(self) -> torch.Tensor:
        return self.tqkv.dense()

    @property
    def wo(self) -> torch.Tensor:
        return self.tout.dense()

    @property
    def wd(self) -> torch.Tensor:
        return self.tdown.dense()

    @property
    def wgu(self) -> torch.Tensor:
        """Gate/up weight as [gate | up] rows (a copy)."""
        t = self.tgu.dense()
        if not self.gu_fused:
            return t
        F2, H = t.shape
        return t.view(F2 // 2, 2, H).transpose(0, 1).reshape(F2, H)


class Decoder:
    """Random-initialised decoder; weights ~ N(0, std), norm weights 1 + N(0, std).
    The vocabulary projection is held tiled (``t_lm_head``); ``lm_head`` gives it
    back row-major (a copy)."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), device="cuda", seed: int = 0, std: float = 0.02):
        self.cfg = cfg
        self.device = torch.device(device)
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)
        self.embed = (torch.randn(cfg.vocab, cfg.hidden, generator=g, device=self.device) * std).to(torch.bfloat16)
        self.layers = [Layer(cfg, g, self.device, std) for _ in range(cfg.layers)]
        self.final_norm = (1.0 + torch.randn(cfg.hidden, generator=g, device=self.device) * std).to(torch.bfloat16)
        self.t_lm_head = tile_weight(
            (torch.randn(cfg.vocab, cfg.hidden, generator=g, device=self.device) * std).to(torch.bfloat16))
        self.sm_scale = cfg.head_dim ** -0.5
        self._ws = {}
        self.attn_ws_used = None   # attention workspace of the last forward (eager or replayed)
        self._ws_retired = []   # outgrown buffers: a captured graph may still point at them
        self._rope = None       # (cos, sin) [positions, head_dim] bf16 tables
        self._graphs: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()

    @property
    def lm_head(self) -> torch.Tensor:
        return self.t_lm_head.dense()

    def _workspace(self, name: str, nbytes: int) -> torch.Tensor:
        """Scratch owned by the model, grown (never while a graph is being
        captured) so that captured kernels keep pointing at live memory."""
        ws = self._ws.get(name)
        if ws is None or ws.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("decoder workspace must be sized before graph capture")
            if ws is not None:
                self._ws_retired.append(ws)
            ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            self._ws[name] = ws
        return ws

    def _rope_rows(self, positions: torch.Tensor, cap: int) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin rows [T, head_dim] of ``positions``, gathered from tables that
        rope_tables computes once for positions [0, cap) -- the same bits as
        computing them per call (every entry depends on its own position only),
        in two gathers instead of a chain of element-wise launches.  A position
        a cache of ``cap`` slots cannot hold is clamped into the table."""
        t = self._rope
        if t is None or t[0].shape[0] < cap:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("rotary tables must be sized before graph capture")
            if t is not None:
                self._ws_retired.append(t)
            cfg = self.cfg
            t = rope_tables(torch.arange(cap, device=self.device), cfg.head_dim, cfg.theta, device=self.device)
            self._rope = t
        idx = positions.clamp(0, t[0].shape[0] - 1)
        return t[0].index_select(0, idx), t[1].index_select(0, idx)

    def _linear(self, x: int, sx: int, M: int, w: TiledWeight, out_dtype=torch.bfloat16) -> torch.Tensor:
        """x (device pointer, row stride sx or RSPX_TILED, M rows) . w^T."""
        L = _lib.lib()
        N, K = w.shape
        need = L.rspx_linear_workspace_bytes(M, N, K)
        ws = self._workspace("linear", max(need, 16))
        out = torch.empty((M, N), dtype=out_dtype, device=self.device)
        _lib.check("rspx_linear", L.rspx_linear(
            x, sx, w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0), M, N, K,
            1 if out_dtype == torch.float32 else 0, ws.data_ptr(), ws.numel(), _lib.stream_ptr(self.device)))
        return out

    def _partials(self, x: int, sx: int, M: int, w: TiledWeight) -> tuple[int, int]:
        """x (device pointer, row stride sx or RSPX_TILED, M rows) . w^T left as
        fp32 chunk partials in the model's partial buffer; returns (pointer,
        chunk count) for a consumer that sums them."""
        L = _lib.lib()
        N, K = w.shape
        S = L.rspx_linear_splits(N, K)
        buf = self._workspace("partials", S * M * N * 4)
        _lib.check("rspx_linear_partials", L.rspx_linear_partials(
            x, sx, w.data_ptr(), w.stride(0), buf.data_ptr(), M, N, K, _lib.stream_ptr(self.device)))
        return buf.data_ptr(), S

    # ------------------------------------------------------------------ forward
    @torch.no_grad()
    def forward(self, ids: torch.Tensor, slots: torch.Tensor, positions: torch.Tensor, cache, P: int,
                msk: torch.Tensor, NN: int) -> torch.Tensor:
        """Run ``T = len(ids)`` tokens through every layer.

        ids [T] int64, slots [T] int32 (cache slot written by each token),
        positions [T] (rotary positions), cache: KVCache whose slots [0, P) are
        the prompt segment and [P, P + NN) the node segment; msk [T, NN] uint8
        (row t may attend to node slot j).  Returns fp32 logits [T, V].
        """
        cfg = self.cfg
        L = _lib.lib()
        dev = self.device
        s = _lib.stream_ptr(dev)
        T = int(ids.shape[0])
        if P < 0 or NN < 0 or P + NN > cache.cap:
            raise ValueError(f"forward: prompt {P} + node segment {NN} exceeds the cache's {cache.cap} slots")
        Hd, HQ, HK, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
        bf = torch.bfloat16
        TILED = _lib.RSPX_TILED
        rows = -(-T // 64) * 64                                   # tiled buffers hold whole 64-row blocks
        x = self.embed.index_select(0, ids)                       # residual stream [T, H]
        y = torch.empty(rows * Hd, dtype=bf, device=dev)          # normalised rows [T, H], tiled
        _lib.check("rspx_rmsnorm", L.rspx_rmsnorm(x.data_ptr(), Hd, self.layers[0].in_norm.data_ptr(), y.data_ptr(),
                                                  TILED, T, Hd, cfg.eps, s))
        cos, sin = self._rope_rows(positions, cache.cap)
        slots32 = slots.to(torch.int32)
        qo = torch.empty((T, HQ, D), dtype=bf, device=dev)
        att = torch.empty(rows * HQ * D, dtype=bf, device=dev)   # attention output [T, HQ D], tiled
        mlp = torch.empty(rows * cfg.ffn, dtype=bf, device=dev)  # SwiGLU output [T, F], tiled when fused
        ws_attn = self._workspace("attn", L.rspx_trie_attn_workspace_bytes(HQ, HK, T, P, D))
        self.attn_ws_used = ws_attn   # its first word flags a wait that gave up (kernels.attention.status_word)
        for li, lay in enumerate(self.layers):
            ck, cv = cache.k[li], cache.v[li]
            qkvp, S = self._partials(y.data_ptr(), TILED, T, lay.tqkv)
            _lib.check("rspx_qkv_rope_cache_partials", L.rspx_qkv_rope_cache_partials(
                qkvp, S, lay.q_norm.data_ptr(), lay.k_norm.data_ptr(), cos.data_ptr(),
                sin.data_ptr(), cos.stride(0), slots32.data_ptr(), cache.cap, ck.data_ptr(), ck.stride(0), ck.stride(1),
                cv.data_ptr(), cv.stride(0), cv.stride(1), qo.data_ptr(), T, HQ, HK, D, cfg.eps, s))
            trie_attn(qo.permute(1, 0, 2), ck[:, :P], cv[:, :P], ck[:, P:P + NN], cv[:, P:P + NN], msk,
                      self.sm_scale, out=att, workspace=ws_attn, out_tiled=True)
            hp, S = self._partials(att.data_ptr(), TILED, T, lay.tout)
            _lib.check("rspx_add_rmsnorm_partials", L.rspx_add_rmsnorm_partials(
                x.data_ptr(), Hd, hp, S, lay.post_norm.data_ptr(), x.data_ptr(), Hd, y.data_ptr(), TILED,
                T, Hd, cfg.eps, s))
            F = cfg.ffn
            if lay.gu_fused:
                _lib.check("rspx_linear_silu", L.rspx_linear_silu(
                    y.data_ptr(), TILED, lay.tgu.data_ptr(), lay.tgu.stride(0), mlp.data_ptr(),
                    TILED, T, 2 * F, Hd, s))
                msx = TILED
            else:
                gu = self._linear(y.data_ptr(), TILED, T, lay.tgu)
                _lib.check("rspx_silu_mul", L.rspx_silu_mul(gu.data_ptr(), gu.stride(0), gu.data_ptr() + 2 * F,
                                                            gu.stride(0), mlp.data_ptr(), F, T, F, s))
                msx = F
            hp, S = self._partials(mlp.data_ptr(), msx, T, lay.tdown)
            nxt = self.layers[li + 1].in_norm if li + 1 < len(self.layers) else self.final_norm
            _lib.check("rspx_add_rmsnorm_partials", L.rspx_add_rmsnorm_partials(
                x.data_ptr(), Hd, hp, S, nxt.data_ptr(), x.data_ptr(), Hd, y.data_ptr(), TILED,
                T, Hd, cfg.eps, s))
        return self._linear(y.data_ptr(), TILED, T, self.t_lm_head, out_dtype=torch.float32)

    # ------------------------------------------------------------------ prompt
    @torch.no_grad()
    def prefill(self, ids: torch.Tensor, cache, chunk: int = 512) -> torch.Tensor:
        """Fill cache slots [0, len(ids)) with the prompt's KV, ``chunk`` tokens per
        forward: a chunk sees the earlier chunks as its prompt segment and
        itself causally as its node segment.  Returns the last row's logits."""
        n = int(ids.shape[0])
        if n > cache.cap:
            raise ValueError(f"prefill: {n} prompt tokens exceed the cache's {cache.cap} slots")
        dev = self.device
        logits = None
        for c0 in range(0, n, chunk):
            c1 = min(n, c0 + chunk)
            T = c1 - c0
            NN = -(-T // 32) * 32
            msk = torch.tril(torch.ones(T, NN, dtype=torch.uint8, device=dev))
            pos = torch.arange(c0, c1, device=dev)
            logits = self.forward(ids[c0:c1], pos.to(torch.int32), pos, cache, c0, msk, NN)
        return logits[-1:]

    # ------------------------------------------------------------------ graphs
    def graphed(self, cache, P: int, T: int, NN: int) -> "GraphedForward":
        """A captured forward for T rows, prompt P and node segment NN over
        ``cache``.  Graphs are kept per cache object (a weak key: they are
        dropped with the cache whose device pointers they hold, so a new cache
        never replays a graph of a freed one)."""
        per_cache = self._graphs.get(cache)
        if per_cache is None:
            per_cache = {}
            self._graphs[cache] = per_cache
        key = (P, T, NN, cache.cap)
        g = per_cache.get(key)
        if g is None:
            g = GraphedForward(self, cache, P, T, NN)
            per_cache[key] = g
        return g

    def release_graphs(self, cache=None) -> None:
        """Drop the captured forwards of ``cache`` (all caches if None) and their memory pools."""
        if cache is None:
            self._graphs.clear()
        else:
            self._graphs.pop(cache, None)


class GraphedForward:
    """Decoder.forward captured once in a HIP graph for fixed (T, P, NN).  The
    row inputs -- tokens, cache slots, rotary positions, mask -- are made inside
    the graph by rspx_step_inputs from a step descriptor [n, base, tokens,
    parents] in device memory, so a call is one host-to-device copy from pinned
    memory and a replay.  Padding rows write their K/V to the last T slots of
    the cache, which no call reads, and attend to node slot 0 only."""

    def __init__(self, model: Decoder, cache, P: int, T: int, NN: int):
        dev = model.device
        self.model = model
        if P + NN > cache.cap - T:
            raise ValueError("KV cache has no room for the graph's scratch slots")
        self.T, self.NN = T, NN
        self.scratch = cache.cap - T
        i32 = torch.int32
        self.desc = torch.zeros(2 + 2 * T, dtype=i32, device=dev)
        self.host = torch.zeros(2 + 2 * T, dtype=i32).pin_memory()
        self.copied = torch.cuda.Event()
        self.ids = torch.zeros(T, dtype=i32, device=dev)
        self.slots = torch.zeros(T, dtype=i32, device=dev)
        self.pos = torch.zeros(T, dtype=i32, device=dev)
        self.msk = torch.zeros(T, NN, dtype=torch.uint8, device=dev)
        # the greedy choice of every row (no excluded vocabulary range), also captured
        self.picks = torch.zeros(T, dtype=torch.int64, device=dev)
        self.picks_host = torch.zeros(T, dtype=torch.int64).pin_memory()
        self.picked = torch.cuda.Event()
        L = _lib.lib()
        vocab = model.cfg.vocab
        # Held by the object: the captured argmax writes here on every replay.
        self.argws = argws = torch.zeros(max(16, L.rspx_argmax_workspace_bytes(T, vocab)), dtype=torch.uint8,
                                         device=dev)

        def body():
            _lib.check("rspx_step_inputs", L.rspx_step_inputs(
                self.desc.data_ptr(), T, P, NN, self.scratch, vocab, self.ids.data_ptr(), self.slots.data_ptr(),
                self.pos.data_ptr(), self.msk.data_ptr(), self.msk.stride(0), _lib.stream_ptr(dev)))
            logits = model.forward(self.ids, self.slots, self.pos, cache, P, self.msk, NN)
            greedy_token(logits, out=self.picks, workspace=argws)
            return logits

        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):  # sizes the workspaces and the allocator pools
            body()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = body()
        # The attention workspace the captured calls use, and a pinned host word
        # for its timeout flag: greedy() copies the flag with the picks.
        self.attn_ws = model.attn_ws_used
        self.flag_host = torch.zeros(1, dtype=torch.int32).pin_memory()

    def run(self, n: int, base: int, tokens, parents) -> torch.Tensor:
        """Replay for the n-node trie ``tokens`` / ``parents`` (parents precede
        children, -1 for a root) after ``base`` committed slots; a 1-token
        forward is a one-node trie.  Returns logits [T, V] (rows n.. padding)."""
        if not 0 <= n <= self.T or base < 0 or base + n > self.NN:
            raise ValueError("trie does not fit the captured forward")
        self.copied.synchronize()  # the previous call's copy is done with the pinned buffer
        h = self.host.numpy()
        h[0], h[1] = n, base
        h[2:2 + n] = tokens
        h[2 + self.T:2 + self.T + n] = parents
        self.desc.copy_(self.host, non_blocking=True)
        self.copied.record()
        self.graph.replay()
        self.model.attn_ws_used = self.attn_ws
        return self.logits

    def greedy(self, n: int) -> list[int]:
        """The greedy tokens of rows [0, n) of the last replay (rspx_argmax_rows
        over the whole vocabulary, taken inside the graph), on the host."""
        self.picks_host[:n].copy_(self.picks[:n], non_blocking=True)
        self.flag_host.copy_(status_word(self.attn_ws), non_blocking=True)
        self.picked.record()
        self.picked.synchronize()
        raise_if_gave_up(int(self.flag_host[0]), self.attn_ws)
        return self.picks_host[:n].tolist()
