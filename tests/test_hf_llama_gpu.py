"""The drop-in on the reference's real caller: a transformers LlamaForCausalLM whose decoder
linears quantize_linears_ swaps for KFLinearInt4 (reference kernelforge/modules.py:51-65), driven
the way the reference's e2e harness drives it (bench/e2e_model.py:85-162,207): a StaticCache, a
prompt forward, then greedy decode eagerly and from a HIP graph of one decode step.

The model is random-init from a small LlamaConfig (no download): 2 layers, hidden 256, 4 query /
2 KV heads of 64, intermediate 768, vocab 1000, fp16, SDPA attention.  Checks:

* quantize_linears_ swaps exactly the 7 decoder linears per layer; embeddings and lm_head stay;
* prompt logits against the same network in fp32 on the CPU with W_hat = q * s from the oracle
  (2e-2 relative rule, same argmax: only activation precision differs);
* greedy tokens from graph replays equal eager StaticCache decode (the reference's check);
* the last decode step's logits against the CPU fp32 model over the whole sequence.
"""

from __future__ import annotations

import pytest
import torch

from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers", reason="transformers does not import here")

DEV = torch.device("cuda")
LAYERS = 2


def _config():
    return transformers.LlamaConfig(vocab_size=1000, hidden_size=256, intermediate_size=768,
                                    num_hidden_layers=LAYERS, num_attention_heads=4, num_key_value_heads=2,
                                    head_dim=64, max_position_embeddings=256, rms_norm_eps=1e-5,
                                    tie_word_embeddings=False, attn_implementation="sdpa")


def _int4_model(seed: int):
    from kernelforge.modules import KFLinearInt4, quantize_linears_

    torch.manual_seed(seed)
    model = transformers.LlamaForCausalLM(_config()).half().to(DEV).eval()
    n = quantize_linears_(model, 128)
    assert n == 7 * LAYERS
    assert sum(isinstance(m, KFLinearInt4) for m in model.modules()) == 7 * LAYERS
    assert isinstance(model.lm_head, torch.nn.Linear) and isinstance(model.model.embed_tokens, torch.nn.Embedding)
    return model


def _cpu_reference(model):
    """The same network in fp32 on the CPU, every INT4 linear replaced by W_hat = q * s (oracle)."""
    from kernelforge.modules import KFLinearInt4

    ref = transformers.LlamaForCausalLM(_config()).float().eval()
    sd = {k: v.float().cpu() for k, v in model.state_dict().items() if not k.endswith((".packed", ".scales"))}
    missing, _ = ref.load_state_dict(sd, strict=False)
    ref_mods = dict(ref.named_modules())
    for name, mod in model.named_modules():
        if isinstance(mod, KFLinearInt4):
            w = o.dequantize_fp32(mod.packed.cpu().numpy(), mod.scales.cpu().numpy(), mod.group_size)
            ref_mods[name].weight.data = torch.from_numpy(w)
            missing.remove(f"{name}.weight")
    assert not missing, f"reference weights not set: {missing}"
    return ref


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).abs().max() / b.abs().max()).item()


def _prompt(n, seed=11):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 1000, (1, n), generator=g)


@torch.no_grad()
def test_prompt_logits_match_cpu_fp32_reference():
    model = _int4_model(0)
    prompt = _prompt(12)
    got = model(prompt.to(DEV)).logits[0]
    ref = _cpu_reference(model)(prompt).logits[0]
    rel = _rel(got, ref)
    assert rel < 2e-2, f"prompt logits rel err {rel:.3e}"
    assert torch.equal(got.float().cpu().argmax(-1), ref.argmax(-1))


@torch.no_grad()
def test_graph_decode_equals_eager_static_cache_and_cpu_reference():
    from transformers import StaticCache

    model = _int4_model(1)
    p, steps = 12, 16
    prompt = _prompt(p, seed=12).to(DEV)

    # Eager decode on a StaticCache: the exact reference for the graph (same cache, masks, kernels).
    cache = StaticCache(config=model.config, max_cache_len=p + steps + 8)
    out = model(prompt, cache_position=torch.arange(p, device=DEV), past_key_values=cache, use_cache=True)
    t = out.logits[:, -1:].argmax(-1)
    eager = [t.item()]
    for i in range(steps):
        out = model(t, cache_position=torch.tensor([p + i], device=DEV), past_key_values=cache, use_cache=True)
        t = out.logits[:, -1:].argmax(-1)
        eager.append(t.item())
    last_eager_logits = out.logits[0, -1].clone()

    # One decode step captured in a HIP graph, replayed with a device-side position.
    cache = StaticCache(config=model.config, max_cache_len=p + steps + 8)
    out = model(prompt, cache_position=torch.arange(p, device=DEV), past_key_values=cache, use_cache=True)
    tok = out.logits[:, -1:].argmax(-1).clone()
    graph_tokens = [tok.item()]
    pos = torch.tensor([p], device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            model(tok, cache_position=pos, past_key_values=cache, use_cache=True)
    torch.cuda.current_stream().wait_stream(side)
    for layer in cache.layers:  # the warm-up calls advanced the cache's own write counter
        if hasattr(layer, "cumulative_length"):
            layer.cumulative_length.fill_(p)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        logits = model(tok, cache_position=pos, past_key_values=cache, use_cache=True).logits
    for _ in range(steps):
        graph.replay()
        tok.copy_(logits[:, -1:].argmax(-1))
        pos.add_(1)
        graph_tokens.append(tok.item())
    torch.cuda.synchronize()
    assert graph_tokens == eager, f"graph {graph_tokens} vs eager {eager}"
    assert torch.equal(logits[0, -1], last_eager_logits)

    # The last step's logits against the CPU fp32 model run over the whole sequence.
    seq = torch.cat([prompt.cpu(), torch.tensor([eager[:steps]])], dim=1)
    ref = _cpu_reference(model)(seq).logits[0, -1]
    rel = _rel(last_eager_logits, ref)
    assert rel < 2e-2, f"decode logits rel err {rel:.3e}"
    assert last_eager_logits.float().cpu().argmax() == ref.argmax()
