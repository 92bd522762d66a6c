"""A TinyLlama-architecture decoder whose linears run on the INT4 path.

Random-initialized (no checkpoints are fetched): 22 layers, hidden 2048, 32 query / 4 KV heads
of dim 64, SwiGLU intermediate 5632, RMSNorm, RoPE, vocab 32000, fp16 activations.  The seven
decoder linears of every layer are ``nn.Linear`` modules named like Hugging Face's
(q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj), so ``quantize_linears_`` swaps
them for ``KFLinearInt4`` exactly as it would in an HF model (reference
kernelforge/modules.py:51-65); embedding and lm_head stay fp16.

``fuse_decoder_linears_`` replaces q|k|v and gate|up by one INT4 module each whose packed rows are
the concatenation of the originals (the packed format is per row, so this is the same format).
For M <= 16 (decode and short prompts: the GEMV and the skinny kernel, whose per-column
arithmetic does not depend on N) the fused results are bit-identical; for larger M the fused and
the separate matrices can take different tiled kernels or split-K counts, which changes only the
fp32 summation order.

Decode follows the reference's graph method (bench/e2e_model.py:85-141): static KV cache,
positions in device tensors, one decode step captured in a HIP graph and replayed; the greedy
token is written back into the graph's input on the device, so replays run back to back.
Attention is plain PyTorch (fp16 matmuls on contiguous operands, fp32 softmax).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn

from kernelforge import ops
from kernelforge.modules import KFLinearInt4


@dataclass
class TinyLlamaConfig:
    vocab: int = 32000
    hidden: int = 2048
    layers: int = 22
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = 64
    intermediate: int = 5632
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_seq: int = 160


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # One fused kernel when x and the weight share a dtype (fp32 accumulation inside).
        return torch.nn.functional.rms_norm(x, (x.shape[-1],), self.weight.to(x.dtype), self.eps)


def _rope_tables(cfg: TinyLlamaConfig, device) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE tables [max_seq, head_dim]: cos, and sin with the sign of rotate-half folded in
    (-sin on the first half), so x * cos + swap_halves(x) * sin is the rotation."""
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float32) / cfg.head_dim))
    t = torch.arange(cfg.max_seq, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    emb = torch.cat([freqs, freqs], dim=-1)
    sin = freqs.sin()
    return emb.cos().to(device), torch.cat([-sin, sin], dim=-1).to(device)


def _rope(x: torch.Tensor, cos: torch.Tensor, sin_signed: torch.Tensor) -> torch.Tensor:
    """x [T, heads, d] rotated by the per-position rows cos / sin_signed [T, 1, d]."""
    h = x.shape[-1] // 2
    return torch.addcmul(x * cos, torch.cat([x[..., h:], x[..., :h]], dim=-1), sin_signed)


def _int4_fused(lin, x, **kw):
    """ops.int4_linear_fused on an INT4 layer (KFLinearInt4 or FusedInt4Linear)."""
    return ops.int4_linear_fused(x, lin.packed, lin.scales, lin.group_size, **kw)


class FusedInt4Linear(nn.Module):
    """Several INT4 linears on the same input as ONE GEMV/GEMM over their concatenated rows.

    Bit-identical to running them separately for M <= 16 (GEMV and skinny kernels compute each
    column independently of N); above that the tiled kernels' choice or split-K count may differ,
    which only reorders fp32 sums.  Returns the per-part outputs.
    """

    def __init__(self, parts: list[KFLinearInt4]):
        super().__init__()
        g = {p.group_size for p in parts}
        k = {p.in_features for p in parts}
        if len(g) != 1 or len(k) != 1 or any(p.bias is not None for p in parts):
            raise ValueError("fused parts need one group size, one in_features and no bias")
        self.group_size = g.pop()
        self.in_features = k.pop()
        self.splits = [p.out_features for p in parts]
        self.register_buffer("packed", torch.cat([p.packed for p in parts], dim=0).contiguous())
        self.register_buffer("scales", torch.cat([p.scales for p in parts], dim=0).contiguous())
        # The parts keep working on the same bytes: their buffers become row slices (contiguous
        # views) of the concatenated ones, so fusing holds no second copy of the weights.
        off = 0
        for p in parts:
            p.packed = self.packed[off:off + p.out_features]
            p.scales = self.scales[off:off + p.out_features]
            off += p.out_features

    def forward(self, x: torch.Tensor) -> list[torch.Tensor]:
        return list(torch.split(self.forward_concat(x), self.splits, dim=-1))

    def forward_concat(self, x: torch.Tensor) -> torch.Tensor:
        """The parts' outputs side by side along the last dimension (one tensor)."""
        return ops.int4_linear(x, self.packed, self.scales, self.group_size)


class Attention(nn.Module):
    def __init__(self, cfg: TinyLlamaConfig):
        super().__init__()
        self.cfg = cfg
        h, d = cfg.hidden, cfg.head_dim
        self.q_proj = nn.Linear(h, cfg.heads * d, bias=False)
        self.k_proj = nn.Linear(h, cfg.kv_heads * d, bias=False)
        self.v_proj = nn.Linear(h, cfg.kv_heads * d, bias=False)
        self.o_proj = nn.Linear(cfg.heads * d, h, bias=False)
        self.qkv: FusedInt4Linear | None = None

    def project(self, x, norm: "RMSNorm | None" = None):
        """(q|k [1, T, (heads + kv_heads) d], v [1, T, kv_heads d]) of x.  With `norm` the layers
        are INT4 and the RMSNorm of x runs inside their GEMV launches (int4_linear_fused)."""
        cfg = self.cfg
        nqk = (cfg.heads + cfg.kv_heads) * cfg.head_dim
        if norm is not None:
            kw = dict(norm_weight=norm.weight, eps=norm.eps)
            if self.qkv is not None:
                y = _int4_fused(self.qkv, x, **kw)
                return y[..., :nqk], y[..., nqk:]
            return (torch.cat([_int4_fused(self.q_proj, x, **kw), _int4_fused(self.k_proj, x, **kw)], dim=-1),
                    _int4_fused(self.v_proj, x, **kw))
        if self.qkv is not None:
            y = self.qkv.forward_concat(x)                               # [1, T, (hq + 2 hkv) d]
            return y[..., :nqk], y[..., nqk:]
        return torch.cat([self.q_proj(x), self.k_proj(x)], dim=-1), self.v_proj(x)

    def core(self, qk, v, pos, cos, sin, cache_k, cache_v, scores):
        """Attention of the new positions over the cache: [1, T, heads d], before o_proj.

        pos int64 [T] positions; cos / sin [T, 1, d] RoPE rows of those positions (sin with the
        rotate-half sign folded in); cache_k / cache_v [kv_heads, max_seq, d] slabs, the key slab
        holding K transposed ([kv_heads, d, max_seq]); scores [kv_heads, rep * T, max_seq] holding
        the additive causal mask repeated for the rep = heads / kv_heads query heads of a KV head,
        overwritten with the scores (see attend)."""
        return self.attend(self.rope_cache(qk, v, pos, cos, sin, cache_k, cache_v), cache_k, cache_v, scores)

    def rope_cache(self, qk, v, pos, cos, sin, cache_k, cache_v):
        """RoPE on q and k, k and v written into the caches at `pos`; returns q [T, heads, d]."""
        cfg = self.cfg
        t = qk.shape[1]
        hq, hkv, d = cfg.heads, cfg.kv_heads, cfg.head_dim
        qk = _rope(qk.view(t, hq + hkv, d), cos, sin)                     # q and k heads together
        q, k = qk[:, :hq], qk[:, hq:]
        cache_k.view(hkv, d, cfg.max_seq).index_copy_(2, pos, k.permute(1, 2, 0))
        cache_v.index_copy_(1, pos, v.view(t, hkv, d).transpose(0, 1))
        return q

    def attend(self, q, cache_k, cache_v, scores):
        """q [T, heads, d] (rotated) over the caches: [1, T, heads d], before o_proj.

        scores: [kv_heads, rep * T, max_seq] holding the mask on entry; the scaled products are
        added to it in place (baddbmm_ with C = D), which spares the copy of the mask into a fresh
        output that an out-of-place baddbmm makes in every layer (same values)."""
        cfg = self.cfg
        t = q.shape[0]
        hq, hkv, d = cfg.heads, cfg.kv_heads, cfg.head_dim
        rep = hq // hkv
        # Query head h reads KV head h // rep: the rep heads of a KV head (and their T positions)
        # form the rows of one batch entry, so K and V are never repeated.
        qg = q.reshape(t, hkv, rep, d).permute(1, 2, 0, 3).reshape(hkv, rep * t, d)
        scores = scores.baddbmm_(qg, cache_k.view(hkv, d, cfg.max_seq), alpha=1.0 / math.sqrt(d))
        probs = torch.softmax(scores, dim=-1)                            # fp32 inside
        out = torch.bmm(probs, cache_v)                                  # [hkv, rep * T, d]
        return out.view(hkv, rep, t, d).permute(2, 0, 1, 3).reshape(1, t, hq * d)

    def forward(self, x, pos, cos, sin, cache_k, cache_v, scores):
        """x [1, T, H] (already normalized); see core for the other arguments."""
        qk, v = self.project(x)
        return self.o_proj(self.core(qk, v, pos, cos, sin, cache_k, cache_v, scores))


class MLP(nn.Module):
    def __init__(self, cfg: TinyLlamaConfig):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden, cfg.intermediate, bias=False)
        self.up_proj = nn.Linear(cfg.hidden, cfg.intermediate, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate, cfg.hidden, bias=False)
        self.gate_up: FusedInt4Linear | None = None

    def project(self, x, norm: "RMSNorm | None" = None):
        """(gate, up) of x; with `norm`, INT4 layers with the RMSNorm inside their GEMV launches."""
        if norm is not None:
            kw = dict(norm_weight=norm.weight, eps=norm.eps)
            if self.gate_up is not None:
                g, u = torch.split(_int4_fused(self.gate_up, x, **kw), self.gate_up.splits, dim=-1)
                return g, u
            return _int4_fused(self.gate_proj, x, **kw), _int4_fused(self.up_proj, x, **kw)
        if self.gate_up is not None:
            g, u = self.gate_up(x)
            return g, u
        return self.gate_proj(x), self.up_proj(x)

    def forward(self, x):
        g, u = self.project(x)
        return self.down_proj(torch.nn.functional.silu(g) * u)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: TinyLlamaConfig):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden, cfg.rms_eps)
        self.self_attn = Attention(cfg)
        self.post_attention_layernorm = RMSNorm(cfg.hidden, cfg.rms_eps)
        self.mlp = MLP(cfg)

    def int4_fusable(self) -> bool:
        """Every linear on the INT4 path without bias: the layer can run the fused launches."""
        a, m = self.self_attn, self.mlp
        qkv = [a.qkv] if a.qkv is not None else [a.q_proj, a.k_proj, a.v_proj]
        gu = [m.gate_up] if m.gate_up is not None else [m.gate_proj, m.up_proj]
        return all(isinstance(p, (KFLinearInt4, FusedInt4Linear)) and getattr(p, "bias", None) is None
                   for p in qkv + gu + [a.o_proj, m.down_proj])

    def forward(self, x, pos, cos, sin, cache_k, cache_v, scores, rope16=None):
        """scores: this layer's mask-filled score buffer (Attention.attend); rope16: the full fp16
        (cos, sin) tables, for the fused q|k|v launch of a decode step."""
        a, m = self.self_attn, self.mlp
        if self.int4_fusable():
            # Four INT4 launches per layer at decode: RMSNorm inside q|k|v and gate|up, the residual
            # adds inside o_proj and down, SiLU-multiply inside down (int4_linear_fused); with
            # q|k|v fused, RoPE and the KV-cache writes inside the q|k|v launch as well.
            ln1 = self.input_layernorm
            if x.shape[1] == 1 and a.qkv is not None and rope16 is not None:
                c = a.cfg
                y = ops.int4_qkv_rope_cache(x, a.qkv.packed, a.qkv.scales, a.qkv.group_size, cos=rope16[0],
                                            sin=rope16[1], pos=pos, cache_k=cache_k, cache_v=cache_v, heads=c.heads,
                                            kv_heads=c.kv_heads, head_dim=c.head_dim, norm_weight=ln1.weight,
                                            eps=ln1.eps)
                out = a.attend(y[..., :c.heads * c.head_dim].view(1, c.heads, c.head_dim), cache_k, cache_v, scores)
            else:
                qk, v = a.project(x, ln1)
                out = a.core(qk, v, pos, cos, sin, cache_k, cache_v, scores)
            x = _int4_fused(a.o_proj, out, residual=x)
            g, u = m.project(x, self.post_attention_layernorm)
            return _int4_fused(m.down_proj, g, up=u, residual=x)
        x = x + a(self.input_layernorm(x), pos, cos, sin, cache_k, cache_v, scores)
        return x + m(self.post_attention_layernorm(x))


class TinyLlama(nn.Module):
    def __init__(self, cfg: TinyLlamaConfig):
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab, cfg.hidden)
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.layers))
        self.norm = RMSNorm(cfg.hidden, cfg.rms_eps)
        self.lm_head = nn.Linear(cfg.hidden, cfg.vocab, bias=False)

    @torch.no_grad()
    def init_random_(self, seed: int = 0) -> "TinyLlama":
        """Seeded N(0, 0.02^2) linear weights and N(0, 1) embeddings, drawn on the module's device."""
        dev = self.embed_tokens.weight.device
        g = torch.Generator(device=dev).manual_seed(seed)
        for mod in self.modules():
            if isinstance(mod, nn.Linear):
                mod.weight.copy_(torch.randn(mod.weight.shape, generator=g, device=dev) * 0.02)
            elif isinstance(mod, nn.Embedding):
                mod.weight.copy_(torch.randn(mod.weight.shape, generator=g, device=dev))
        return self


    def new_cache(self, device, dtype=torch.float16) -> torch.Tensor:
        """KV cache [layers, 2, kv_heads, max_seq, head_dim]; each layer's key slab holds K
        transposed (read as [kv_heads, head_dim, max_seq]), the value slab V as laid out."""
        c = self.cfg
        return torch.zeros(c.layers, 2, c.kv_heads, c.max_seq, c.head_dim, device=device, dtype=dtype)

    @torch.no_grad()
    def forward(self, tokens, pos, cache, rope, mask, logits_fp32: bool = True):
        """tokens int64 [T]; pos int64 [T]; mask [T, max_seq] additive (0 / -inf); returns logits of
        the last position, [vocab], fp32 (or the lm_head's own dtype with logits_fp32=False).
        Inference only (no autograd)."""
        cos, sin = rope
        x = self.embed_tokens(tokens).unsqueeze(0)
        # Per-token inputs shared by every layer: RoPE rows of the positions, and every layer's
        # score buffer filled with the mask (repeated for the query heads that share a KV head) by
        # one copy; each layer adds its scores to its own buffer in place.
        c_ = self.cfg
        t, rep = tokens.numel(), c_.heads // c_.kv_heads
        scores = mask.to(x.dtype).view(1, 1, 1, t, c_.max_seq).expand(c_.layers, c_.kv_heads, rep, t, c_.max_seq)
        # contiguous() materializes the broadcast (reshape alone would stay a stride-0 view at T = 1).
        scores = scores.contiguous().view(c_.layers, c_.kv_heads, rep * t, c_.max_seq)
        rope16 = (cos.to(x.dtype), sin.to(x.dtype)) if x.is_cuda and tokens.numel() == 1 else None
        # The per-position rows are only needed by layers that apply RoPE in torch.
        if rope16 is not None and all(ly.int4_fusable() and ly.self_attn.qkv is not None for ly in self.layers):
            c = s = None
        else:
            c, s = cos[pos].to(x.dtype).unsqueeze(1), sin[pos].to(x.dtype).unsqueeze(1)
        for i, layer in enumerate(self.layers):
            x = layer(x, pos, c, s, cache[i, 0], cache[i, 1], scores[i], rope16)
        x = self.norm(x[:, -1:])
        logits = self.lm_head(x).view(-1)
        return logits.float() if logits_fp32 else logits


def causal_mask(pos: torch.Tensor, max_seq: int) -> torch.Tensor:
    """[T, max_seq] additive mask: 0 where key index <= query position, -inf elsewhere."""
    keys = torch.arange(max_seq, device=pos.device)
    return torch.where(keys[None, :] <= pos[:, None], 0.0, float("-inf")).float()


@torch.no_grad()
def fuse_decoder_linears_(model: TinyLlama) -> int:
    """Fuses q|k|v and gate|up INT4 linears of every layer (after quantize_linears_)."""
    n = 0
    for layer in model.layers:
        a, m = layer.self_attn, layer.mlp
        if all(isinstance(p, KFLinearInt4) for p in (a.q_proj, a.k_proj, a.v_proj)):
            a.qkv = FusedInt4Linear([a.q_proj, a.k_proj, a.v_proj])
            n += 1
        if all(isinstance(p, KFLinearInt4) for p in (m.gate_proj, m.up_proj)):
            m.gate_up = FusedInt4Linear([m.gate_proj, m.up_proj])
            n += 1
    return n


class GraphDecoder:
    """Greedy decode with one HIP-graph-captured step (static cache, device-side positions).

    The captured step reads the current token and position from static device tensors, runs
    the model, writes argmax into the token buffer and the output history, and advances the
    position, so replays need no host round trip.  The host keeps its own count of the position
    and refuses (ValueError) a prefill, capture or decode whose steps would write past the last
    history / cache slot (max_seq - 1): a step at position p writes history[p + 1].
    """

    def __init__(self, model: TinyLlama, device):
        self.model, self.device = model, device
        cfg = model.cfg
        # fp16 tables: the per-token casts in the model's forward are then no-ops.
        self.rope = tuple(t.to(model.embed_tokens.weight.dtype) for t in _rope_tables(cfg, device))
        self.cache = model.new_cache(device)
        self.token = torch.zeros(1, dtype=torch.long, device=device)
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self.history = torch.zeros(cfg.max_seq, dtype=torch.long, device=device)
        # The decode step's additive mask [1, max_seq] in the activation dtype: 0 for the cache
        # slots up to the current position, -inf past them.  Prefill opens the prompt's slots and
        # the first decode position's; every step opens the next one, so the mask is never built
        # anew.
        self.mask = torch.full((1, cfg.max_seq), float("-inf"), dtype=model.embed_tokens.weight.dtype, device=device)
        self.graph = None
        self.host_pos = 0

    def _reserve(self, steps: int, what: str) -> None:
        """Raises unless `steps` more steps from the current position stay inside max_seq."""
        last = self.model.cfg.max_seq - 1
        if self.host_pos + steps > last:
            raise ValueError(f"{what}: {steps} step(s) from position {self.host_pos} would write position "
                             f"{self.host_pos + steps}, past max_seq - 1 = {last}")

    def _step(self):
        if self.token.is_cuda:
            # argmax over the fp16 logits, pos += 1, history / token / mask updates: one launch.
            logits = self.model(self.token, self.pos, self.cache, self.rope, self.mask, logits_fp32=False)
            ops.decode_argmax_step(logits, self.token, self.pos, self.history, self.mask)
            return
        logits = self.model(self.token, self.pos, self.cache, self.rope, self.mask)
        nxt = torch.argmax(logits).view(1)
        self.pos.add_(1)
        self.history.index_copy_(0, self.pos, nxt)
        self.token.copy_(nxt)
        self.mask.index_fill_(1, self.pos, 0.0)

    def prefill(self, prompt: torch.Tensor) -> None:
        """Runs the prompt eagerly; leaves the first generated token in self.token."""
        t = prompt.numel()
        if not 0 < t < self.model.cfg.max_seq:
            raise ValueError(f"prefill: a prompt of {t} tokens needs 0 < t < max_seq = {self.model.cfg.max_seq}")
        pos = torch.arange(t, device=self.device)
        self.cache.zero_()
        logits = self.model(prompt, pos, self.cache, self.rope, causal_mask(pos, self.model.cfg.max_seq))
        self.history.zero_()
        self.history[:t] = prompt
        self.token.copy_(torch.argmax(logits).view(1))
        self.history[t] = self.token[0]
        self.pos.fill_(t)
        self.mask.fill_(float("-inf"))
        self.mask[:, :t + 1] = 0.0
        self.host_pos = t

    def capture(self) -> None:
        self._reserve(2, "capture (two warm-up steps)")
        saved = (self.cache.clone(), self.token.clone(), self.pos.clone(), self.history.clone(), self.mask.clone())
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        # capture ran warm-up steps; restore the state after prefill
        self.cache.copy_(saved[0])
        self.token.copy_(saved[1])
        self.pos.copy_(saved[2])
        self.history.copy_(saved[3])
        self.mask.copy_(saved[4])

    def decode(self, steps: int, use_graph: bool = True) -> torch.Tensor:
        self._reserve(steps, "decode")
        self.host_pos += steps
        for _ in range(steps):
            if use_graph:
                self.graph.replay()
            else:
                self._step()
        return self.history

    def generated(self, prompt_len: int, steps: int) -> torch.Tensor:
        return self.history[prompt_len:prompt_len + steps + 1].clone()


def build_int4_model(cfg: TinyLlamaConfig, device, seed: int = 0, group_size: int = 128,
                     fuse: bool = True) -> TinyLlama:
    """Random-init TinyLlama on `device` in fp16 with every decoder linear on the INT4 path."""
    from kernelforge.modules import quantize_linears_

    with torch.device(device):
        model = TinyLlama(cfg)
    model.init_random_(seed).half()
    quantize_linears_(model, group_size)
    if fuse:
        fuse_decoder_linears_(model)
    return model.eval()
