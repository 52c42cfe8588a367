"""Fused q/k RMSNorm + rotary embedding + KV store (HIP sd_qk_norm_rope_store) against the oracle.

Covers Qwen3Attention.pre_attn after the qkv split (nanovllm/models/qwen3.py:89-96: q_norm / k_norm,
rotary_emb) and the store Attention.forward does next (nanovllm/layers/attention.py:62-63).

Tolerance. The kernel follows the reference's eager operations one by one; the only freedom is the order of
the 128-term fp32 sum of squares. Hence:
* rotation only (no norm), v-cache rows and every case whose sum of squares is exact in any order
  (inputs on a coarse grid): bit-exact;
* random inputs with the norm: at least 99.5% of elements bit-exact, and every element within
  2^-6 * (|y1| + |y2|) of the oracle for its rotation pair (y1, y2), about one bf16 unit at the pair's scale;
* k_cache rows are bitwise the kernel's own k output; nothing else in the caches is written.
"""
import pytest
import torch

from nanovllm_amd.layers.attention import Attention, store_kvcache
from nanovllm_amd.layers.rotary_embedding import RotaryEmbedding, qk_norm_rope_store
from nanovllm_amd.utils.context import reset_context, set_context
from oracle import qk_norm_rope as onr

pytestmark = pytest.mark.gpu

D = 128


def _bits(x):
    return x.contiguous().view(torch.int16)


def _case(device, N, Hq, Hkv, seed, P=40960, base=1e6, NB=64, bs=256, pad_frac=0.1, grid=False):
    """One qkv tensor (q / k / v are its split views), positions, weights, table, caches and slots."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    W = (Hq + 2 * Hkv) * D
    if grid:    # values k/4, |k| <= 8: squares and their sums are exact in fp32 in any order
        qkv = (torch.randint(-8, 9, (N, W), generator=g).float() / 4).to(torch.bfloat16)
    else:
        qkv = (torch.randn(N, W, generator=g) * 3).to(torch.bfloat16)
    pos = torch.randint(0, P, (N,), generator=g)
    qw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cs = onr.rope_cache(D, P, base)
    slots = torch.randperm(NB * bs, generator=g)[:N].to(torch.int32)
    npad = int(pad_frac * N)
    if npad:
        slots[torch.randperm(N, generator=g)[:npad]] = -1
    c = dict(qkv=qkv, pos=pos, qw=qw, kw=kw, cs=cs, slots=slots, N=N, Hq=Hq, Hkv=Hkv, NB=NB, bs=bs)
    c["dev"] = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in c.items()}
    return c


def _split(qkv, N, Hq, Hkv):
    q = qkv[:, :Hq * D].view(N, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D)
    return q, k, v


def _run_both(c, norm=True, store=True):
    N, Hq, Hkv, NB, bs = c["N"], c["Hq"], c["Hkv"], c["NB"], c["bs"]
    d = c["dev"]
    q, k, v = _split(d["qkv"], N, Hq, Hkv)
    kc = torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16, device=q.device) if store else None
    vc = torch.zeros_like(kc) if store else None
    qo, ko = qk_norm_rope_store(d["pos"], q, k, v, d["qw"] if norm else None, d["kw"] if norm else None, 1e-6,
                                d["cs"], kc, vc, d["slots"] if store else None)
    torch.cuda.synchronize()
    cq, ck, cv = _split(c["qkv"], N, Hq, Hkv)
    ekc = torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16) if store else None
    evc = torch.zeros_like(ekc) if store else None
    eq, ek = onr.qk_norm_rope_store(cq, ck, cv, c["pos"], c["qw"] if norm else None, c["kw"] if norm else None,
                                    1e-6, c["cs"], ekc, evc, c["slots"] if store else None)
    return dict(q=qo.cpu(), k=ko.cpu(), kc=None if kc is None else kc.cpu(), vc=None if vc is None else vc.cpu(),
                eq=eq, ek=ek, ekc=ekc, evc=evc, v=cv)


def _check_close(got, ref, what):
    """>= 99.5% bit-exact, and within 2^-6 * (|y1| + |y2|) of the oracle per rotation pair."""
    exact = (_bits(got) == _bits(ref)).float().mean().item()
    r = ref.double()
    pair = r[..., :D // 2].abs() + r[..., D // 2:].abs()
    bound = torch.cat((pair, pair), -1) * 2 ** -6
    err = (got.double() - r).abs()
    assert bool((err <= bound).all()), f"{what}: max err {float(err.max())}, exact {exact:.5f}"
    assert exact >= 0.995, f"{what}: only {exact:.5f} bit-exact"
    return exact


def _check_caches(res, slots, Hkv):
    """v rows bitwise; k rows bitwise the kernel's own k; untouched slots stay zero."""
    kflat, vflat = res["kc"].view(-1, Hkv, D), res["vc"].view(-1, Hkv, D)
    valid = slots >= 0
    s = slots[valid].long()
    assert torch.equal(_bits(vflat[s]), _bits(res["v"][valid]))
    assert torch.equal(_bits(kflat[s]), _bits(res["k"][valid]))
    touched = (kflat != 0).flatten(1).any(-1) | (vflat != 0).flatten(1).any(-1)
    assert int(touched.sum()) <= int(valid.sum())
    keep = torch.ones(kflat.size(0), dtype=torch.bool)
    keep[s] = False
    assert not touched[keep].any()


# (28, 4): 36 heads per token, so the 8-lane groups of one wave mix q, k and v heads of two tokens.
# (5, 128, 16) and (3, 120, 8): more than 1024 lanes a token (160 and 136 heads with v), so a token's heads
# span two workgroups
@pytest.mark.parametrize("N,Hq,Hkv", [(1, 32, 8), (7, 32, 8), (64, 32, 8), (2048, 32, 8), (20, 16, 8), (33, 28, 4),
                                     (5, 128, 16), (3, 120, 8)])
def test_norm_rope_store_vs_oracle(device, N, Hq, Hkv):
    print(f"case N={N} Hq={Hq} Hkv={Hkv}", flush=True)
    c = _case(device, N, Hq, Hkv, seed=N + Hq)
    res = _run_both(c)
    eq = _check_close(res["q"], res["eq"], "q")
    ek = _check_close(res["k"], res["ek"], "k")
    print(f"bit-exact fraction q {eq:.6f} k {ek:.6f}", flush=True)
    _check_caches(res, c["slots"], Hkv)


def test_norm_bitexact_when_sum_is_exact(device):
    """On a coarse grid the sum of squares is exact in any order, so the kernel matches bit for bit: this
    pins the correctly rounded 1/sqrt, the two roundings of the norm and the rotation arithmetic."""
    c = _case(device, 512, 32, 8, seed=11, grid=True)
    res = _run_both(c)
    assert torch.equal(_bits(res["q"]), _bits(res["eq"]))
    assert torch.equal(_bits(res["k"]), _bits(res["ek"]))
    _check_caches(res, c["slots"], 8)


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (28, 4)])
def test_rope_only_bitexact(device, Hq, Hkv):
    """No norm (models with a qkv bias) and no store: the rotation alone is bit-exact."""
    c = _case(device, 300, Hq, Hkv, seed=12)
    res = _run_both(c, norm=False, store=False)
    assert torch.equal(_bits(res["q"]), _bits(res["eq"]))
    assert torch.equal(_bits(res["k"]), _bits(res["ek"]))


def test_rope_only_with_store_bitexact(device):
    """Rotation without the norm but with the store (qkv-bias models in the fused path): bit-exact, and the
    caches hold the rotated k and the unchanged v."""
    c = _case(device, 129, 28, 4, seed=19)
    res = _run_both(c, norm=False, store=True)
    assert torch.equal(_bits(res["q"]), _bits(res["eq"]))
    assert torch.equal(_bits(res["k"]), _bits(res["ek"]))
    assert torch.equal(_bits(res["kc"]), _bits(res["ekc"])) and torch.equal(_bits(res["vc"]), _bits(res["evc"]))
    _check_caches(res, c["slots"], 4)


def test_in_place_and_no_k_out(device):
    c = _case(device, 100, 32, 8, seed=13)
    res = _run_both(c)
    d = c["dev"]
    qkv = d["qkv"].clone()
    q, k, v = _split(qkv, 100, 32, 8)
    kc = torch.zeros(c["NB"], c["bs"], 8, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    qo, ko = qk_norm_rope_store(d["pos"], q, k, v, d["qw"], d["kw"], 1e-6, d["cs"], kc, vc, d["slots"], q_out=q,
                                k_out=k)
    assert qo.data_ptr() == q.data_ptr() and ko.data_ptr() == k.data_ptr()
    torch.cuda.synchronize()
    assert torch.equal(_bits(q.cpu()), _bits(res["q"])) and torch.equal(_bits(k.cpu()), _bits(res["k"]))
    assert torch.equal(_bits(kc.cpu()), _bits(res["kc"])) and torch.equal(_bits(vc.cpu()), _bits(res["vc"]))
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(kc)
    q2, _, v2 = _split(d["qkv"], 100, 32, 8)
    k2 = d["qkv"][:, 32 * D:40 * D].view(100, 8, D)
    qo2, ko2 = qk_norm_rope_store(d["pos"], q2, k2, v2, d["qw"], d["kw"], 1e-6, d["cs"], kc2, vc2, d["slots"],
                                  write_k=False)
    torch.cuda.synchronize()
    assert ko2 is None
    assert torch.equal(_bits(qo2.cpu()), _bits(res["q"])) and torch.equal(_bits(kc2.cpu()), _bits(res["kc"]))


def test_bad_positions_and_slots(device):
    """Out-of-range positions give NaN rows for that token only; slots >= num_slots and -1 are skipped."""
    c = _case(device, 16, 32, 8, seed=14, P=1000, NB=2, bs=16, pad_frac=0)
    d = c["dev"]
    pos = d["pos"].clone()
    pos[3], pos[9] = -1, 1000
    slots = d["slots"].clone()
    slots[5], slots[6] = 32, -1                      # 32 == num_slots
    q, k, v = _split(d["qkv"], 16, 32, 8)
    kc = torch.zeros(2, 16, 8, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    qo, ko = qk_norm_rope_store(pos, q, k, v, d["qw"], d["kw"], 1e-6, d["cs"], kc, vc, slots)
    torch.cuda.synchronize()
    bad = torch.zeros(16, dtype=torch.bool)
    bad[[3, 9]] = True
    assert qo[bad.to(device)].isnan().all() and ko[bad.to(device)].isnan().all()
    assert not qo[~bad.to(device)].isnan().any() and not ko[~bad.to(device)].isnan().any()
    written = (vc.view(32, -1) != 0).any(-1).cpu()
    expect = torch.zeros(32, dtype=torch.bool)
    for t in range(16):
        s = int(slots[t])
        if 0 <= s < 32:
            expect[s] = True
    assert torch.equal(written, expect)


def test_argument_errors(device):
    c = _case(device, 4, 32, 8, seed=15)
    d = c["dev"]
    q, k, v = _split(d["qkv"], 4, 32, 8)
    with pytest.raises(ValueError):
        qk_norm_rope_store(d["pos"], q, k, v, d["qw"], None, 1e-6, d["cs"])
    with pytest.raises(ValueError):
        qk_norm_rope_store(d["pos"].int(), q, k, v, None, None, 1e-6, d["cs"])
    qq = torch.zeros(4, 32, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        qk_norm_rope_store(d["pos"], qq, qq[:, :8], None, None, None, 1e-6, d["cs"])


def test_graph_capture_replays(device):
    """Captured once, replayed with new rows, positions and slots written in place: every replay matches the
    eager call on the same inputs."""
    c = _case(device, 64, 32, 8, seed=16)
    d = c["dev"]
    qkv, pos, slots = d["qkv"].clone(), d["pos"].clone(), d["slots"].clone()
    q, k, v = _split(qkv, 64, 32, 8)
    kc = torch.zeros(c["NB"], c["bs"], 8, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    qo = torch.empty(64, 32, D, dtype=torch.bfloat16, device=device)
    ko = torch.empty(64, 8, D, dtype=torch.bfloat16, device=device)
    qk_norm_rope_store(pos, q, k, v, d["qw"], d["kw"], 1e-6, d["cs"], kc, vc, slots, q_out=qo, k_out=ko)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qk_norm_rope_store(pos, q, k, v, d["qw"], d["kw"], 1e-6, d["cs"], kc, vc, slots, q_out=qo, k_out=ko)
    for r in range(3):
        nc = _case(device, 64, 32, 8, seed=100 + r)
        qkv.copy_(nc["dev"]["qkv"])
        pos.copy_(nc["dev"]["pos"])
        slots.copy_(nc["dev"]["slots"])
        kc.zero_()
        vc.zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = (qo.cpu(), ko.cpu(), kc.cpu(), vc.cpu())
        kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
        eq, ek = qk_norm_rope_store(pos, q, k, v, d["qw"], d["kw"], 1e-6, d["cs"], kc2, vc2, slots)
        torch.cuda.synchronize()
        assert torch.equal(_bits(got[0]), _bits(eq.cpu())) and torch.equal(_bits(got[1]), _bits(ek.cpu()))
        assert torch.equal(_bits(got[2]), _bits(kc2.cpu())) and torch.equal(_bits(got[3]), _bits(vc2.cpu()))


def test_rotary_module_drop_in(device):
    """RotaryEmbedding(head, rotary_dim, max_pos, base).forward(positions, q, k) against the oracle rotation
    with the module's own table (bit-exact), and its table against the oracle's closed form."""
    rope = RotaryEmbedding(D, D, 8192, 1e6).to(device)
    g = torch.Generator().manual_seed(17)
    q = torch.randn(50, 32 * D, generator=g).to(torch.bfloat16)
    k = torch.randn(50, 8 * D, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, 8192, (50,), generator=g)
    qo, ko = rope(pos.to(device), q.to(device), k.to(device))
    assert qo.shape == q.shape and ko.shape == k.shape
    cs = rope.cos_sin_cache.reshape(8192, D).cpu()
    assert torch.allclose(cs, onr.rope_cache(D, 8192, 1e6), atol=2e-6)
    eq, ek = onr.rotary(pos, q.view(50, 32, D), k.view(50, 8, D), cs)
    torch.cuda.synchronize()
    assert torch.equal(_bits(qo.cpu().view(50, 32, D)), _bits(eq))
    assert torch.equal(_bits(ko.cpu().view(50, 8, D)), _bits(ek))


def test_attention_after_fused_store_equals_unfused(device):
    """Decode step: fused pre_attn (store included) + Attention.forward(kv_stored=True) gives bitwise the
    output of norm/rope without store + Attention.forward storing itself."""
    B, n, Hq, Hkv, bs, NB = 4, 5, 32, 8, 256, 16
    N = B * n
    c = _case(device, N, Hq, Hkv, seed=18, NB=NB, bs=bs, pad_frac=0)
    d = c["dev"]
    q, k, v = _split(d["qkv"], N, Hq, Hkv)
    lens = torch.tensor([300, 512, 777, 1024], dtype=torch.int32, device=device)
    tables = torch.arange(B * 4, dtype=torch.int32, device=device).view(B, 4)
    pos_list = [p for L in lens.tolist() for p in range(L - n, L)]
    pos = torch.tensor(pos_list, dtype=torch.int64, device=device)
    tab = tables.cpu()
    slots = torch.tensor([int(tab[i // n, p // bs]) * bs + p % bs for i, p in enumerate(pos_list)],
                         dtype=torch.int32, device=device)
    base = torch.randn(NB, bs, Hkv, D, device=device).to(torch.bfloat16)
    outs = []
    for fused in (True, False):
        attn = Attention(Hq, D, D ** -0.5, Hkv)
        attn.k_cache, attn.v_cache = base.clone(), base.clone()
        set_context(False, slot_mapping=slots, context_lens=lens, block_tables=tables)
        if fused:
            qo, _ = qk_norm_rope_store(pos, q, k, v, d["qw"], d["kw"], 1e-6, d["cs"], attn.k_cache, attn.v_cache,
                                       slots, write_k=False)
            o = attn(qo, None, None, kv_stored=True)
        else:
            qo, ko = qk_norm_rope_store(pos, q, k, v, d["qw"], d["kw"], 1e-6, d["cs"])
            store_kvcache(ko, v, attn.k_cache, attn.v_cache, slots)
            o = attn(qo, ko, v, kv_stored=True)
        reset_context()
        outs.append((o.cpu(), attn.k_cache.cpu(), attn.v_cache.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(_bits(a), _bits(b))
