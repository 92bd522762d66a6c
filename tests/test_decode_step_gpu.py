"""kf_decode_argmax_step (ops.decode_argmax_step): the greedy step of the graph-captured decoder.

The index must be torch.argmax's on the same fp16 logits (first index of the maximum, NaN above
every number), and the bookkeeping must be the decoder's: pos += 1, token = idx, history[pos] =
idx and mask[pos] = 0 while pos < max_seq, nothing written past the buffers' ends.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kernelforge import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _state(max_seq: int, p: int):
    token = torch.full((1,), -1, dtype=torch.int64, device=DEV)
    pos = torch.full((1,), p, dtype=torch.int64, device=DEV)
    history = torch.full((max_seq + 8,), -7, dtype=torch.int64, device=DEV)  # 8 guard entries
    mask = torch.full((max_seq + 8,), float("-inf"), dtype=torch.float16, device=DEV)
    return token, pos, history, mask


def _step(logits, max_seq=64, p=10):
    token, pos, history, mask = _state(max_seq, p)
    ops.decode_argmax_step(logits, token, pos, history[:max_seq], mask[:max_seq])
    torch.cuda.synchronize()
    return token, pos, history, mask


def _logits(n, seed):
    return torch.from_numpy(np.random.default_rng(seed).standard_normal(n).astype(np.float16)).to(DEV)


@pytest.mark.parametrize("n", [1, 7, 8, 1001, 32000, 151936])
def test_argmax_matches_torch(n):
    for seed in range(3):
        x = _logits(n, seed + n)
        token, pos, history, mask = _step(x)
        want = int(torch.argmax(x))
        assert int(token) == want == int(history[11]), (n, seed)
        assert int(pos) == 11 and float(mask[11]) == 0.0


def test_ties_nan_and_infinities_follow_torch():
    n = 32000
    cases = []
    x = _logits(n, 1)
    top = float(x.max())
    for idx in (31999, 5000, 17, 5001):  # equal maxima: the smallest index wins
        x[idx] = top + 2
    cases.append(x)
    y = _logits(n, 2)
    y[[40, 9000, 30000]] = float("nan")  # the first NaN wins
    cases.append(y)
    cases.append(torch.full((n,), float("-inf"), dtype=torch.float16, device=DEV))  # index 0
    z = _logits(n, 3)
    z[123] = float("inf")
    z[77] = float("inf")
    cases.append(z)
    w = torch.zeros(n, dtype=torch.float16, device=DEV)
    w[::2] = -0.0  # +0 and -0 are equal: index 0
    cases.append(w)
    for i, c in enumerate(cases):
        token, _, _, _ = _step(c)
        assert int(token) == int(torch.argmax(c)), f"case {i}"


def test_misaligned_logits_take_the_scalar_path():
    buf = _logits(32008, 9)
    x = buf[1:32001]
    assert x.data_ptr() % 16 == 2
    token, _, _, _ = _step(x)
    assert int(token) == int(torch.argmax(x))


def test_bookkeeping_stops_at_the_end_of_the_cache():
    x = _logits(512, 4)
    want = int(torch.argmax(x))
    max_seq = 16
    token, pos, history, mask = _step(x, max_seq=max_seq, p=max_seq - 2)  # writes slot 15
    assert int(pos) == max_seq - 1 and int(history[max_seq - 1]) == want and float(mask[max_seq - 1]) == 0.0
    token, pos, history, mask = _step(x, max_seq=max_seq, p=max_seq - 1)  # p = 16: no history / mask write
    assert int(pos) == max_seq and int(token) == want
    assert bool((history == -7).all()) and bool(torch.isinf(mask).all())


def test_graph_replays_advance_like_eager_steps():
    max_seq = 32
    xs = torch.stack([_logits(4096, 50 + i) for i in range(6)])
    cur = torch.empty(4096, dtype=torch.float16, device=DEV)
    token, pos, history, mask = _state(max_seq, 3)
    h, m = history[:max_seq], mask[:max_seq]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.decode_argmax_step(cur, token, pos, h, m)
    torch.cuda.current_stream().wait_stream(side)
    pos.fill_(3)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.decode_argmax_step(cur, token, pos, h, m)
    for i in range(6):
        cur.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert int(pos) == 4 + i and int(token) == int(torch.argmax(xs[i])) == int(h[4 + i])
    assert bool((m[4:10] == 0).all()) and bool(torch.isinf(m[10:]).all())


def test_argument_errors():
    x = _logits(64, 1)
    token, pos, history, mask = _state(16, 0)
    with pytest.raises(TypeError):
        ops.decode_argmax_step(x.float(), token, pos, history, mask)
    with pytest.raises(ValueError, match="pos"):
        ops.decode_argmax_step(x, token, pos.int(), history, mask)
    with pytest.raises(ValueError, match="mask"):
        ops.decode_argmax_step(x, token, pos, history[:16], mask[:15])
