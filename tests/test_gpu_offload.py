"""The offload dispatch hooks (bin/offload.py:137-451, bin/test_cache.py
restated): every copy mode and the host-side LRU give outputs identical to the
all-resident kernel, at decode-shaped and prefill-shaped calls."""
import numpy as np
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu
E, H, I, K = 32, 2048, 512, 8


@pytest.fixture(scope="module")
def models(dev):
    import moe
    import synth
    ref = moe.MoEExperts(E, H, I, device=dev)
    synth.fill_experts(ref, seed=2, recipe="blockq")
    host = moe.MoEExperts(E, H, I, device="cpu")
    for n in ("w13_weight", "w2_weight", "w13_scale_inv", "w2_scale_inv"):
        setattr(host, n, getattr(ref, n).cpu().pin_memory())
    host._layer_index = 0
    return ref, host


def _call(ref, host, tokens, seed, dev):
    import moe
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((tokens, H), generator=g).to(torch.bfloat16).to(dev)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(tokens)]).to(dev)
    w = torch.rand((tokens, K), generator=g).to(dev)
    w = w / w.sum(-1, keepdim=True)
    want = moe.MoEExperts._stock_forward(ref, x, ids, w)
    return x, ids, w, want


@pytest.mark.parametrize("mode", ["direct", "gather"])
def test_copy_modes_match_resident(lib, dev, models, mode):
    import offload
    ref, host = models
    offload.COPY_MODE = mode
    try:
        for step, tokens in enumerate([1, 5, 1, 17]):
            x, ids, w, want = _call(ref, host, tokens, step, dev)
            say(f"offload: {mode} tokens={tokens}")
            got = offload.offloaded_forward(host, x, ids, w)
            assert torch.equal(got, want)
    finally:
        offload.COPY_MODE = "direct"


def test_hybrid_gather_borrows_device_cache(lib, dev, models):
    import devcache
    import offload
    ref, host = models
    devcache.init_dev_cache(host, dev, 16)
    try:
        for step in range(6):                      # populate the device cache
            _, ids, _, _ = _call(ref, host, 1, 50 + step, dev)
            devcache.dev_resolve_and_fetch(host, ids)
        before = dict(offload.STATS)
        stamp = host._dc_stamp.clone()
        x, ids, w, want = _call(ref, host, 9, 99, dev)
        got = offload.offloaded_forward(host, x, ids, w)
        assert torch.equal(got, want)
        assert offload.STATS["gather_hits"] > before["gather_hits"]
        assert torch.equal(stamp, host._dc_stamp)        # read-only use
    finally:
        for a in [a for a in vars(host) if a.startswith("_dc_")]:
            delattr(host, a)


def test_host_lru_and_fallbacks(lib, dev, models):
    import offload
    ref, host = models
    for cap in (8, 12, E):
        offload._init_cache(host, dev, cap)
        say(f"offload: host LRU cap {cap}")
        for step in range(12):
            tokens = 1 if step % 3 else 5
            x, ids, w, want = _call(ref, host, tokens, 1000 + step, dev)
            got = offload.offloaded_forward(host, x, ids, w)
            assert torch.equal(got, want), f"cap {cap} step {step}"
    for a in ("_cap", "_cache_w13", "_cache_w2", "_cache_s13", "_cache_s2", "_slot_of", "_lru",
              "_free"):
        delattr(host, a)


def test_graphstub_and_none_modes_run(lib, dev, models):
    import offload
    ref, host = models
    x, ids, w, _ = _call(ref, host, 1, 7, dev)
    for mode in ("graphstub", "none"):
        offload.COPY_MODE = mode
        try:
            out = offload.offloaded_forward(host, x, ids, w)
            assert out.shape == (1, H) and torch.isfinite(out.float()).all()
        finally:
            offload.COPY_MODE = "direct"
