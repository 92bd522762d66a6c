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
* the last decode step's logits against the CPU fp32 model over the whole sequence;
* group_sibling_linears_ (q/k/v and gate/up of every layer in one grouped launch each): the
  same logits and tokens as the ungrouped model, bit for bit, eager and from the graph.
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


def _decode(model, prompt, steps: int):
    """Greedy decode the reference's way (bench/e2e_model.py:85-162): eager on a StaticCache, then
    from a HIP graph of one decode step replayed with a device-side position.  Returns the eager
    tokens, the graph tokens, and the last step's eager and graph logits."""
    from transformers import StaticCache

    p = prompt.shape[1]
    cache = StaticCache(config=model.config, max_cache_len=p + steps + 8)
    out = model(prompt, cache_position=torch.arange(p, device=DEV), past_key_values=cache, use_cache=True)
    t = out.logits[:, -1:].argmax(-1)
    eager = [t.item()]
    for i in range(steps):
        out = model(t, cache_position=torch.tensor([p + i], device=DEV), past_key_values=cache, use_cache=True)
        t = out.logits[:, -1:].argmax(-1)
        eager.append(t.item())
    last_eager_logits = out.logits[0, -1].clone()

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
    return eager, graph_tokens, last_eager_logits, logits[0, -1].clone()


@torch.no_grad()
def test_graph_decode_equals_eager_static_cache_and_cpu_reference():
    model = _int4_model(1)
    steps = 16
    prompt = _prompt(12, seed=12).to(DEV)
    eager, graph_tokens, last_eager_logits, last_graph_logits = _decode(model, prompt, steps)
    assert graph_tokens == eager, f"graph {graph_tokens} vs eager {eager}"
    assert torch.equal(last_graph_logits, last_eager_logits)

    # The last step's logits against the CPU fp32 model run over the whole sequence.
    seq = torch.cat([prompt.cpu(), torch.tensor([eager[:steps]])], dim=1)
    ref = _cpu_reference(model)(seq).logits[0, -1]
    rel = _rel(last_eager_logits, ref)
    assert rel < 2e-2, f"decode logits rel err {rel:.3e}"
    assert last_eager_logits.float().cpu().argmax() == ref.argmax()


@torch.no_grad()
def test_grouped_siblings_equal_ungrouped_model(monkeypatch):
    """group_sibling_linears_ on the HF model: q/k/v and gate/up of every layer share one grouped
    launch (counted on an eager decode step); prompt logits, eager and graph-decoded tokens and the
    last logits equal the ungrouped model's bit for bit, and the CPU fp32 model within 2e-2."""
    from kernelforge import modules, ops

    plain, grouped = _int4_model(3), _int4_model(3)
    assert modules.group_sibling_linears_(grouped) == 2 * LAYERS
    prompt = _prompt(12, seed=13).to(DEV)
    assert torch.equal(grouped(prompt).logits, plain(prompt).logits)

    calls = []
    real = ops.int4_linear_grouped
    monkeypatch.setattr(ops, "int4_linear_grouped", lambda *a, **k: calls.append(len(a[0])) or real(*a, **k))
    grouped(prompt[:, :1])
    assert calls == [3, 2] * LAYERS, calls
    monkeypatch.setattr(ops, "int4_linear_grouped", real)

    steps = 12
    want = _decode(plain, prompt, steps)
    got = _decode(grouped, prompt, steps)
    assert got[0] == want[0] and got[1] == want[1] == want[0], (got[:2], want[:2])
    assert torch.equal(got[2], want[2]) and torch.equal(got[3], want[3])
    seq = torch.cat([prompt.cpu(), torch.tensor([got[0][:steps]])], dim=1)
    ref = _cpu_reference(grouped)(seq).logits[0, -1]
    assert _rel(got[2], ref) < 2e-2 and got[2].float().cpu().argmax() == ref.argmax()
