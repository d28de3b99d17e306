"""The forward and the packed varlen pass under HIP graph capture (torch.cuda.CUDAGraph): every launch is stream
ordered, nothing synchronises and nothing clears memory with hipMemsetAsync, so a captured call replays exactly.
Each replay runs after unrelated eager work on the same buffers' neighbours and must equal the eager result bit for
bit.  The reference's sageattn_varlen reads cu_seqlens back to the host and cannot be captured."""
import pytest
import torch

import cdna4_sage
import sageattention

pytestmark = pytest.mark.gpu


def _replays_match(fn, args, eager, n=4):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(*args)                       # warm-up on the capture stream (plans and lazy state)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        out = fn(*args)
    for i in range(n):
        noise = torch.randn(1 << 20, device=args[0].device).sum()    # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        assert torch.isfinite(noise)


def test_forward_graph_replays(dev):
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 24, 4608, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    fn = lambda a, b, c: sageattention.sageattn(a, b, c, tensor_layout="HND")   # noqa: E731
    eager = fn(q, k, v).clone()
    _replays_match(fn, (q, k, v), eager)
    q2, k2, v2 = (torch.randn(2, 8, 3000, 64, generator=g).to(torch.float16).to(dev) for _ in range(3))
    fn2 = lambda a, b, c: cdna4_sage.attention(a, b, c, "HND", is_causal=True)   # noqa: E731
    _replays_match(fn2, (q2, k2, v2), fn2(q2, k2, v2).clone())


def test_varlen_graph_replays(dev):
    g = torch.Generator().manual_seed(1)
    lens = [1500, 700, 2200, 64]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)
    T = sum(lens)
    q, k, v = (torch.randn(T, 16, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    fn = lambda a, b, c: cdna4_sage.attention_varlen(a, b, c, cu, cu, max(lens), max(lens), is_causal=True)  # noqa: E731
    _replays_match(fn, (q, k, v), fn(q, k, v).clone())
