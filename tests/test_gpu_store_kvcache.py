"""KV-cache scatter on the GPU (HIP sd_store_kvcache) against the oracle: bit-exact.

Covers the reference contract nanovllm/layers/attention.py:33-40: -1 slots skipped, strided value rows
(the qkv split), row-stride asserts, hipGraph capture with padding rows, the unaligned element path.
"""
import pytest
import torch

from nanovllm_amd.layers.attention import store_kvcache
from oracle import kvcache as okv

pytestmark = pytest.mark.gpu


def _bits(x):
    return x.view(torch.int16)


def _inputs(device, N, Hkv, D, NB, bs, pad_frac, seed, strided=True):
    g = torch.Generator(device=device).manual_seed(seed)
    if strided:   # k and v as views of a fused qkv row, like Qwen3Attention.pre_attn
        qkv = torch.randn(N, (4 + 2) * Hkv * D, device=device, generator=g).to(torch.bfloat16)
        key = qkv[:, 4 * Hkv * D:5 * Hkv * D].view(N, Hkv, D)
        value = qkv[:, 5 * Hkv * D:].view(N, Hkv, D)
    else:
        key = torch.randn(N, Hkv, D, device=device, generator=g).to(torch.bfloat16)
        value = torch.randn(N, Hkv, D, device=device, generator=g).to(torch.bfloat16)
    slots = torch.randperm(NB * bs, device=device, generator=g)[:N].to(torch.int32)
    npad = int(pad_frac * N)
    if npad:
        slots[torch.randperm(N, device=device, generator=g)[:npad]] = -1
    return key, value, slots


def test_store_small_vs_oracle_bitexact(device):
    N, Hkv, D, NB, bs = 300, 8, 128, 16, 256
    key, value, slots = _inputs(device, N, Hkv, D, NB, bs, 0.1, 0)
    kc = torch.randn(NB, bs, Hkv, D, device=device).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    ek, ev = kc.cpu(), vc.cpu()
    store_kvcache(key, value, kc, vc, slots)
    okv.store_kvcache(key.cpu(), value.cpu(), ek, ev, slots.cpu())
    torch.cuda.synchronize()
    assert torch.equal(_bits(kc.cpu()), _bits(ek)) and torch.equal(_bits(vc.cpu()), _bits(ev))


def test_store_config2_full_size(device):
    """Qwen3-8B KV shapes: 2048 rows into a 4096-block x 256-slot cache, 10% padding slots (-1)."""
    N, Hkv, D, NB, bs = 2048, 8, 128, 4096, 256
    key, value, slots = _inputs(device, N, Hkv, D, NB, bs, 0.1, 1)
    kc = torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    store_kvcache(key, value, kc, vc, slots)
    valid = slots >= 0
    s = slots[valid].long()
    assert torch.equal(_bits(kc.view(-1, Hkv * D)[s]), _bits(key.reshape(N, -1)[valid]))
    assert torch.equal(_bits(vc.view(-1, Hkv * D)[s]), _bits(value.reshape(N, -1)[valid]))
    # nothing else was written: exactly the valid slots hold non-zero rows
    touched = (kc.view(-1, Hkv * D) != 0).any(-1)
    assert int(touched.sum()) == int(valid.sum())
    assert bool(touched[s].all())


def test_store_contiguous_and_unaligned_paths(device):
    Hkv, D, NB, bs = 2, 10, 4, 32          # row of 20 elements: 40 B, not a multiple of 16 B -> element path
    N = 40
    key, value, slots = _inputs(device, N, Hkv, D, NB, bs, 0.2, 2, strided=False)
    for H, Dh in ((Hkv, D), (8, 128)):
        if (H, Dh) != (Hkv, D):
            key, value, slots = _inputs(device, N, H, Dh, NB, bs, 0.2, 3, strided=False)
        kc = torch.randn(NB, bs, H, Dh, device=device).to(torch.bfloat16)
        vc = torch.randn_like(kc)
        ek, ev = kc.cpu(), vc.cpu()
        store_kvcache(key, value, kc, vc, slots)
        okv.store_kvcache(key.cpu(), value.cpu(), ek, ev, slots.cpu())
        assert torch.equal(_bits(kc.cpu()), _bits(ek)) and torch.equal(_bits(vc.cpu()), _bits(ev))


def test_store_graph_capture_with_padding(device):
    """Captured once, replayed with new slot mappings (padding rows -1), each replay checked bit-exact."""
    N, Hkv, D, NB, bs = 64, 8, 128, 8, 256
    key = torch.zeros(N, Hkv, D, dtype=torch.bfloat16, device=device)
    value = torch.zeros_like(key)
    slots = torch.full((N,), -1, dtype=torch.int32, device=device)
    kc = torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    store_kvcache(key, value, kc, vc, slots)     # warm up outside the capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        store_kvcache(key, value, kc, vc, slots)
    for it in range(4):
        k2, v2, s2 = _inputs(device, N, Hkv, D, NB, bs, 0.25, 10 + it, strided=False)
        key.copy_(k2)
        value.copy_(v2)
        slots.copy_(s2)
        ek, ev = kc.cpu(), vc.cpu()
        graph.replay()
        torch.cuda.synchronize()
        okv.store_kvcache(k2.cpu(), v2.cpu(), ek, ev, s2.cpu())
        assert torch.equal(_bits(kc.cpu()), _bits(ek)) and torch.equal(_bits(vc.cpu()), _bits(ev)), it


def test_store_rejects_bad_strides(device):
    key = torch.zeros(4, 8, 128, dtype=torch.bfloat16, device=device)
    kc = torch.zeros(2, 256, 8, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        store_kvcache(key.transpose(1, 2).contiguous().transpose(1, 2), key, kc, kc.clone(),
                      torch.zeros(4, dtype=torch.int32, device=device))
    with pytest.raises(ValueError):
        store_kvcache(key, key, kc, kc.clone(), torch.zeros(3, dtype=torch.int32, device=device))
