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


@torch.no_grad()
def test_logits_match_cpu_fp32_reference():
    """First-token logits of the INT4 fp16 model vs the same network in fp32 on the CPU with
    W_hat = q * s from the oracle (only the activation precision differs)."""
    cfg = _small_cfg()
    model = tl.build_int4_model(cfg, DEV, seed=2, fuse=False)  # fusion itself: test above
    prompt = _prompt(12, cfg.vocab)
    pos = torch.arange(12, device=DEV)
    got = model(prompt, pos, model.new_cache(DEV), tl._rope_tables(cfg, DEV), tl.causal_mask(pos, cfg.max_seq))

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
    cpu = torch.device("cpu")
    ref = ref_model(prompt.cpu(), pos.cpu(), ref_model.new_cache(cpu, torch.float32), tl._rope_tables(cfg, cpu),
                    tl.causal_mask(pos.cpu(), cfg.max_seq))
    got = got.cpu()
    rel = (got - ref).abs().max() / ref.abs().max()
    assert rel < 2e-2, f"logits rel err {rel:.3e}"
    assert torch.argmax(got) == torch.argmax(ref)


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
