"""End-to-end decode of a random-init TinyLlama-architecture model on the INT4 path (BASELINE
config 5), checked the reference's way (graph decode == eager decode, bench/e2e_model.py:144-162,207)
plus a CPU fp32 reference forward built from the oracle's dequantized weights."""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from kernelforge import tinyllama as tl
from kernelforge.modules import KFLinearInt4
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _small_cfg(layers=2, max_seq=48):
    return dataclasses.replace(tl.TinyLlamaConfig(), layers=layers, max_seq=max_seq)


def _prompt(n, vocab, seed=3):
    return torch.from_numpy(np.random.default_rng(seed).integers(0, vocab, n)).to(DEV)


@torch.no_grad()
def test_fused_qkv_gateup_bit_identical():
    cfg = _small_cfg()
    model = tl.build_int4_model(cfg, DEV, seed=1, fuse=False)
    prompt = _prompt(8, cfg.vocab)
    pos = torch.arange(8, device=DEV)
    rope = tl._rope_tables(cfg, DEV)
    mask = tl.causal_mask(pos, cfg.max_seq)
    a = model(prompt, pos, model.new_cache(DEV), rope, mask)
    assert tl.fuse_decoder_linears_(model) == 2 * cfg.layers
    b = model(prompt, pos, model.new_cache(DEV), rope, mask)
    assert torch.equal(a, b)


def _cpu_fp32_reference(model, cfg):
    """The same network in fp32 on the CPU with W_hat = q * s from the oracle for every INT4 linear
    (only the activation precision differs from the GPU model)."""
    ref_model = tl.TinyLlama(cfg).float()
    sd = {k: v.float().cpu() for k, v in model.state_dict().items() if "packed" not in k and "scales" not in k}
    ref_model.load_state_dict(sd, strict=False)
    ref_mods = dict(ref_model.named_modules())
    n_int4 = 0
    for name, mod in model.named_modules():
        if isinstance(mod, KFLinearInt4):
            w = o.dequantize_fp32(mod.packed.cpu().numpy(), mod.scales.cpu().numpy(), mod.group_size)
            ref_mods[name].weight.data = torch.from_numpy(w)
            n_int4 += 1
    assert n_int4 == 7 * cfg.layers
    return ref_model


def _cpu_logits(ref_model, cfg, tokens):
    cpu = torch.device("cpu")
    pos = torch.arange(tokens.numel())
    return ref_model(tokens.cpu(), pos, ref_model.new_cache(cpu, torch.float32), tl._rope_tables(cfg, cpu),
                     tl.causal_mask(pos, cfg.max_seq))


def _rel(a, b):
    return ((a.float().cpu() - b.float().cpu()).abs().max() / b.float().cpu().abs().max()).item()


@torch.no_grad()
def test_logits_match_cpu_fp32_reference():
    """First-token logits of the INT4 fp16 model (prefill, M = 12 rows through int4_linear) vs the
    CPU fp32 model on the oracle's W_hat."""
    cfg = _small_cfg()
    model = tl.build_int4_model(cfg, DEV, seed=2, fuse=False)  # fusion itself: test above
    prompt = _prompt(12, cfg.vocab)
    pos = torch.arange(12, device=DEV)
    got = model(prompt, pos, model.new_cache(DEV), tl._rope_tables(cfg, DEV), tl.causal_mask(pos, cfg.max_seq))
    ref = _cpu_logits(_cpu_fp32_reference(model, cfg), cfg, prompt)
    rel = _rel(got, ref)
    assert rel < 2e-2, f"logits rel err {rel:.3e}"
    assert torch.argmax(got.cpu()) == torch.argmax(ref)


@torch.no_grad()
@pytest.mark.parametrize("steps", [1, 3])
def test_fused_decode_matches_cpu_fp32_reference(steps):
    """The decode path the e2e benchmark runs, checked against an independent reference: a
    2-layer fuse=True model prefills 12 tokens, then decodes `steps` tokens one at a time, each
    through the fused launches (int4_qkv_rope_cache with the RMSNorm prologue and the cache
    writes, gate|up with RMSNorm, down with SwiGLU, the residual adds in o_proj and down).  The
    logits of every decode step are compared with the CPU fp32 model (oracle W_hat) run over the
    whole sequence so far (2e-2 rule, same argmax), and with a fuse=False model stepped the same
    way (torch composition around int4_linear)."""
    cfg = _small_cfg()
    fused = tl.build_int4_model(cfg, DEV, seed=6, fuse=True)
    plain = tl.build_int4_model(cfg, DEV, seed=6, fuse=False)
    assert torch.equal(fused.layers[0].self_attn.q_proj.packed, plain.layers[0].self_attn.q_proj.packed)
    assert all(ly.int4_fusable() and ly.self_attn.qkv is not None for ly in fused.layers)
    ref_model = _cpu_fp32_reference(fused, cfg)
    prompt = _prompt(12, cfg.vocab, seed=8)
    rope = tl._rope_tables(cfg, DEV)
    caches = {}
    for name, model in (("fused", fused), ("plain", plain)):
        caches[name] = model.new_cache(DEV)
        pos = torch.arange(12, device=DEV)
        model(prompt, pos, caches[name], rope, tl.causal_mask(pos, cfg.max_seq))
    tokens = prompt.clone()
    nxt = torch.from_numpy(np.random.default_rng(9).integers(0, cfg.vocab, steps)).to(DEV)
    for i in range(steps):
        tok = nxt[i:i + 1]
        p1 = torch.tensor([12 + i], device=DEV)
        got = {name: model(tok, p1, caches[name], rope, tl.causal_mask(p1, cfg.max_seq))
               for name, model in (("fused", fused), ("plain", plain))}
        tokens = torch.cat([tokens, tok])
        ref = _cpu_logits(ref_model, cfg, tokens)
        for name in ("fused", "plain"):
            rel = _rel(got[name], ref)
            assert rel < 2e-2, f"{name} decode step {i}: logits rel err {rel:.3e}"
            assert torch.argmax(got[name].cpu()) == torch.argmax(ref), f"{name} decode step {i}: argmax"
        assert _rel(got["fused"], got["plain"]) < 1e-2, f"fused vs unfused decode step {i}"


@torch.no_grad()
def test_graph_decoder_refuses_positions_past_the_cache():
    """GraphDecoder keeps a host count of the position and raises before a step would write
    past the history / cache (max_seq), instead of launching an out-of-range index."""
    cfg = _small_cfg(layers=1, max_seq=24)
    model = tl.build_int4_model(cfg, DEV, seed=4, fuse=True)
    dec = tl.GraphDecoder(model, DEV)
    dec.prefill(_prompt(16, cfg.vocab, seed=5))
    dec.capture()
    dec.decode(cfg.max_seq - 1 - 16)  # the last allowed step writes history[max_seq - 1]
    with pytest.raises(ValueError, match="max_seq"):
        dec.decode(1)
    with pytest.raises(ValueError, match="max_seq"):
        dec.prefill(_prompt(cfg.max_seq, cfg.vocab))


@torch.no_grad()
@pytest.mark.parametrize("layers", [2, 22])
def test_graph_decode_equals_eager(layers):
    """Greedy tokens from graph replays equal eager decode on the same static cache (reference
    check, bench/e2e_model.py:207)."""
    cfg = _small_cfg(layers=layers, max_seq=16 + 40)
    model = tl.build_int4_model(cfg, DEV, seed=4, fuse=True)
    prompt = _prompt(16, cfg.vocab, seed=5)
    dec = tl.GraphDecoder(model, DEV)
    dec.prefill(prompt)
    dec.decode(32, use_graph=False)
    eager = dec.generated(16, 32)
    dec.prefill(prompt)
    dec.capture()
    dec.decode(32, use_graph=True)
    torch.cuda.synchronize()
    graph = dec.generated(16, 32)
    assert torch.equal(eager, graph), f"eager {eager.tolist()} vs graph {graph.tolist()}"
    assert (graph >= 0).all() and (graph < cfg.vocab).all()
