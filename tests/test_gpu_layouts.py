"""Attention over paged caches whose block size and query-heads-per-KV-head ratio differ from the Qwen3-8B
defaults (block 256, 32 q / 8 kv heads), against the fp32 oracle (max-abs <= 2e-2, mean-abs <= 2e-3).

Block sizes: 32 (one key tile per block), 96 (not a power of two: the tile -> block mapping divides instead
of shifting), 512 (sixteen tiles per block id). Ratios g = Hq / Hkv: 1, 2, 4, 8, 16, 32 (g = 16 and 32 split
a verify step's rows over several query groups; the prefill q-block then holds 8 or 4 positions).
Decode / verify goes through sd_paged_decode; varlen batches mix prefill chunks (more than 16 queries) and
short rows (at most 16 queries, the residue kernel) in one sd_varlen_attention launch.
"""
import numpy as np
import pytest
import torch

from nanovllm_amd.layers.attention import paged_decode_attention, varlen_attention
from oracle import attention as oatt
from attn_cases import error_stats, paged_cache, queries

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
D = 128
# (block_size, Hq, Hkv)
CASES = [(32, 8, 8), (96, 32, 8), (512, 16, 8), (96, 16, 1), (32, 32, 2), (512, 32, 1)]


def _check(out, ref, what):
    mx, mean = error_stats(out, ref)
    print(f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (what, mx, mean)


@pytest.mark.parametrize("bs,Hq,Hkv", CASES)
def test_decode_block_sizes_and_head_ratios(device, bs, Hq, Hkv):
    """Contexts at and around the block edges (a multiple of 32 for every block size here)."""
    ctx = [1, 31, 95, 96, 97, 511, 513, 1500, 3000]
    B = len(ctx)
    for n in (1, 5, 9):
        kc, vc, tables = paged_cache(device, ctx, Hkv, D, bs=bs, seed=bs + n)
        q = queries(device, B * n, Hq, D, seed=bs + n + 1).view(B, n, Hq, D)
        lens = torch.tensor(ctx, dtype=torch.int32, device=device)
        out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
        ref = oatt.paged_decode_attention(q.cpu(), kc.cpu(), vc.cpu(), lens.cpu(), tables.cpu(), D ** -0.5)
        _check(out.view(B, n, Hq, D), ref, f"decode bs={bs} Hq={Hq} Hkv={Hkv} n={n}")


@pytest.mark.parametrize("bs,Hq,Hkv", CASES)
def test_varlen_block_sizes_and_head_ratios(device, bs, Hq, Hkv):
    """Prefill chunks after cached prefixes (a chunk of 17 queries is the shortest prefill run) and verify /
    decode rows in one launch."""
    pairs = [(5, 600), (300, 300), (129, 1153), (1, 97), (700, 1500), (17, 200), (16, 16), (64, 545)]
    lq = [a for a, _ in pairs]
    lk = [b for _, b in pairs]
    kc, vc, tables = paged_cache(device, lk, Hkv, D, bs=bs, seed=bs + Hq)
    q = queries(device, sum(lq), Hq, D, seed=bs + Hq + 1)
    cu_q = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32, device=device)
    cu_k = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32, device=device)
    out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
    ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q.cpu(), cu_k.cpu(), D ** -0.5, tables.cpu())
    _check(out, ref, f"varlen bs={bs} Hq={Hq} Hkv={Hkv}")


def _aliased_cache(device, B, W, Hkv, bs, NB=48, seed=0):
    """A small cache of NB blocks behind block tables of width W whose entries alias them at random: contexts
    of W * bs keys without W * B blocks of memory."""
    g = torch.Generator(device=device).manual_seed(seed)
    kc = torch.randn(NB, bs, Hkv, D, device=device, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, bs, Hkv, D, device=device, generator=g).to(torch.bfloat16)
    tables = torch.randint(0, NB, (B, W), device=device, generator=g, dtype=torch.int32)
    return kc, vc, tables


@pytest.mark.parametrize("W", [1130, 2048])
@pytest.mark.parametrize("B", [2, 16, 64])
def test_decode_tables_past_1024_blocks(device, B, W):
    """Block size 32 with contexts of 33-36 K keys (tables of 1130 blocks, more than half the 2048 block ids a
    work item stages in LDS) and up to 65 536 keys (tables of 2048 blocks: the limit, the last context using the
    last id slot and the last tile of its last block); B = 2: the one-residue stream kernel, 16: four-wave
    workgroups with partials, 64: eight-wave workgroups merging in LDS."""
    bs, Hq, Hkv, n = 32, 32, 8, 5
    kc, vc, tables = _aliased_cache(device, B, W, Hkv, bs, seed=B + W)
    rnd = np.random.default_rng(B + W)
    ctx = rnd.integers(W * bs - 3000, W * bs + 1, B).tolist()
    ctx[0] = W * bs
    q = queries(device, B * n, Hq, D, seed=B + 1).view(B, n, Hq, D)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
    rows = list(range(min(B, 4)))   # the oracle on a few sequences
    ref = oatt.paged_decode_attention(q[rows].cpu(), kc.cpu(), vc.cpu(), lens[rows].cpu(), tables[rows].cpu(),
                                      D ** -0.5)
    _check(out.view(B, n, Hq, D)[rows], ref, f"B={B}, tables of {W} blocks")


@pytest.mark.parametrize("W", [1130, 2048])
def test_varlen_tables_past_1024_blocks(device, W):
    """A 40-query prefill chunk after a cached prefix and a 5-query verify row, block size 32, 1130-block tables
    (34 000 and 35 000 keys) and 2048-block ones (the limit: 65 536 keys for the verify row, its last tile in
    the last id slot), in one mixed launch and as a prefill-only call."""
    bs, Hq, Hkv = 32, 32, 8
    kc, vc, tables = _aliased_cache(device, 2, W, Hkv, bs, seed=7 + W)
    lq, lk = ([5, 40], [35000, 34040]) if W == 1130 else ([5, 40], [W * bs, W * bs - 1000])
    q = queries(device, sum(lq), Hq, D, seed=8)
    cu_q = torch.tensor([0, 5, 45], dtype=torch.int32, device=device)
    cu_k = torch.tensor([0, lk[0], lk[0] + lk[1]], dtype=torch.int32, device=device)
    out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
    ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q.cpu(), cu_k.cpu(), D ** -0.5, tables.cpu())
    _check(out, ref, f"varlen, tables of {W} blocks")
    # the chunk alone (a prefill-only call) gives the same rows bitwise
    cu_q1 = torch.tensor([0, lq[1]], dtype=torch.int32, device=device)
    cu_k1 = torch.tensor([0, lk[1]], dtype=torch.int32, device=device)
    alone = varlen_attention(q[5:], kc, vc, cu_q1, cu_k1, lq[1], lk[1], D ** -0.5, tables[1:])
    assert torch.equal(alone, out[5:])
