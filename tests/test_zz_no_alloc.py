"""moe_fp8_moe_forward_noalloc, the allocation-free forward, against
moe_fp8_moe_forward_ex with a caller's workspace on the same arguments.

Both run the same kernels, so the bar is bit-identical bf16 outputs.  Two
calls in a row share the library's per-GPU scratch array: a large grouped
call (100 tokens) and then a smaller decode call (1 token, GEMV), so the
second call runs over what the first left in the array.  The noalloc calls
make no allocation through torch's caching allocator either.
"""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu

E, H, I, K = 64, 2048, 512, 8


def _experts(dev):
    import synth
    g = torch.Generator(device=dev).manual_seed(11)
    w13, s13 = synth.quantize_blocks(torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02)
    w2, s2 = synth.quantize_blocks(torch.randn((E, H, I), generator=g, device=dev) * 0.02)
    return w13, s13, w2, s2


def _route(T, seed, dev, ids_dtype, w_dtype):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)])
    w = rng.random((T, K)) + 0.05
    w = w / w.sum(-1, keepdims=True)
    return (torch.tensor(ids, dtype=ids_dtype, device=dev),
            torch.tensor(w, dtype=torch.float32, device=dev).to(w_dtype))


def _allocs(dev) -> int:
    return torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0)


def test_noalloc_forward_equals_workspace_forward(lib, dev):
    w13, s13, w2, s2 = _experts(dev)
    cases = [  # (tokens, ids dtype, weights dtype, residual) -- the second call is smaller
        (100, torch.int64, torch.float32, True),
        (1, torch.int32, torch.bfloat16, False),
    ]
    for n, (T, idt, wdt, with_res) in enumerate(cases):
        import synth
        x = synth.hidden_states(20 + n, T).to(dev)
        res = synth.hidden_states(40 + n, T).to(dev) if with_res else None
        ids, w = _route(T, 30 + n, dev, idt, wdt)
        ws = torch.empty(lib.fp8_moe_workspace(T, K, E, H, I), dtype=torch.uint8, device=dev)
        want = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
        got = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize(dev)
        say(f"noalloc: call {n + 1}, {T} tokens, ids {idt}, weights {wdt}, residual {with_res}")
        lib.fp8_moe_forward(x, ids, w, w13, s13, w2, s2, want, ws, residual=res)
        before = _allocs(dev)
        lib.fp8_moe_forward_noalloc(x, ids, w, w13, s13, w2, s2, got, residual=res)
        torch.cuda.synchronize(dev)
        assert _allocs(dev) == before, "the noalloc forward allocated through torch"
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
            f"call {n + 1}: {(got != want).sum().item()} of {got.numel()} outputs differ"


def test_noalloc_forward_refuses_an_oversized_call_on_the_gpu(lib, dev):
    import hipfetch
    T = 512                                   # ~35 MiB of workspace, past the 16 MiB array
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    ids = torch.zeros((T, K), dtype=torch.int32, device=dev)
    w = torch.zeros((T, K), dtype=torch.float32, device=dev)
    w13, s13, w2, s2 = (torch.zeros((1, 2 * I, H), dtype=torch.uint8, device=dev),
                        torch.ones((1, 8, 16), device=dev),
                        torch.zeros((1, H, I), dtype=torch.uint8, device=dev),
                        torch.ones((1, 16, 4), device=dev))
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    say("noalloc: 512-token call refused")
    with pytest.raises(hipfetch.NativeError, match="more than the"):
        lib.fp8_moe_forward_noalloc(x, ids, w, w13, s13, w2, s2, out)
