"""The whole-model decode / verify step runner and greedy speculative decoding at model scale on the GPU.

* DecodeStepRunner: a 3-layer Qwen3-8B-shaped stack (random bf16 weights) replayed from its (n, batch bucket)
  graph equals the same body run eagerly, bitwise, in the hidden states and every layer's KV cache, for plain
  decode (n = 1) and verify (n = 5) steps with a padded batch (the reference's graph / eager pairs,
  tests/test_greedy.py MUST_MATCH).
* Greedy spec == plain: the same stack in its row-invariant mode (sd_linear projections, sd_rms_norm norms)
  with the real 151,936 x 4,096 LM head through one GEMM for every consumer (lm_head_sample for the prompts'
  first tokens and plain decode, lm_head_verify for verify steps). Prompts are prefilled by the mixed-step
  runner, then decoded 40 steps plainly and with k = 4 guesses (the plain run's tokens, some replaced by
  wrong ones so that steps accept everything, nothing and runs in between). The tokens are identical: the
  property the reference checks end to end only up to bf16 near-ties (tests/test_greedy.py:1-20), held here
  bitwise because no kernel on the path computes a row differently with the batch.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from nanovllm_amd.engine.decode_step import DecodeStepRunner
from nanovllm_amd.engine.mixed_step import MixedStepRunner
from nanovllm_amd.engine.qwen3_segments import Qwen3Segments
from nanovllm_amd.layers.lm_head import LMHeadVerifier, lm_head_sample, lm_head_verify

pytestmark = pytest.mark.gpu

HQ, HKV, D, BLOCK, K = 32, 8, 128, 256, 4
LAYERS = 3


class Seq:
    """The fields the metadata builders read (nanovllm_amd.engine.metadata)."""

    def __init__(self, tokens, block_table):
        self.token_ids = list(tokens)
        self.block_table = list(block_table)
        self.draft_token_ids = []
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = len(tokens)
        self.is_prefill = True

    @property
    def num_tokens(self):
        return len(self.token_ids)

    @property
    def last_token(self):
        return self.token_ids[-1]

    def __len__(self):
        return len(self.token_ids)


def _caches(device, NB):
    return [SimpleNamespace(k_cache=torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16, device=device),
                            v_cache=torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16, device=device))
            for _ in range(LAYERS)]


def test_decode_runner_graph_equals_eager(device):
    model = Qwen3Segments(num_layers=LAYERS, device=device, seed=4, max_tokens=320)
    rng = np.random.default_rng(4)
    B, W = 3, 6
    ctx = [300, 1000, 1400]
    NB = B * W + 2
    graph_layers, eager_layers = _caches(device, NB), _caches(device, NB)
    g = torch.Generator(device=device).manual_seed(5)
    for a, b in zip(graph_layers, eager_layers):    # a filled cache (the prompts' KV)
        a.k_cache.copy_(torch.randn(a.k_cache.shape, device=device, generator=g).to(torch.bfloat16))
        a.v_cache.copy_(torch.randn(a.v_cache.shape, device=device, generator=g).to(torch.bfloat16))
        b.k_cache.copy_(a.k_cache)
        b.v_cache.copy_(a.v_cache)
    perm = rng.permutation(NB)
    runners = [DecodeStepRunner(layers, model, HQ, HKV, D, D ** -0.5, BLOCK, table_width=W, max_batch=64)
               for layers in (graph_layers, eager_layers)]
    for step, n in enumerate([5, 1, 5]):
        seqs = []
        for b in range(B):
            s = Seq(rng.integers(0, 151936, size=ctx[b] + step).tolist(), perm[b * W:(b + 1) * W].tolist())
            s.is_prefill = False
            s.draft_token_ids = rng.integers(0, 151936, size=n - 1).tolist()
            seqs.append(s)
        outs = []
        for r, use_graph in zip(runners, (True, False)):
            layout = r.prepare(seqs, n)
            outs.append(r.run(layout, use_graph=use_graph).clone())
        torch.cuda.synchronize()
        print(f"step {step}: n={n}, bucket {layout['B']}, hidden |mean| {outs[1].float().abs().mean().item():.3f}",
              flush=True)
        assert torch.isfinite(outs[1].float()).all()
        assert torch.equal(outs[0], outs[1]), f"step {step}: graph hidden states differ from the eager body"
        for i, (a, b) in enumerate(zip(graph_layers, eager_layers)):
            assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.v_cache, b.v_cache), f"layer {i} caches"
    assert set(runners[0].graphs) == {(5, 4), (1, 4)}


def _prefill(mixed, model, head, seqs, device):
    """All prompts in one mixed step (prefill chunks only); returns each prompt's first token (greedy)."""
    layout = mixed.prepare(seqs, 0)
    ids = torch.zeros(layout["N"], dtype=torch.int64)
    ids[:layout["n"]] = torch.tensor(layout["input_ids"])
    model.input_ids[:layout["N"]] = ids.to(device)
    mixed.run(layout)
    idx = torch.tensor(layout["logits_indices"], dtype=torch.int64, device=device)
    return lm_head_sample(model.hidden_out, head, torch.zeros(len(seqs), device=device), logits_indices=idx).tolist()


def _start(prompts, tables, mixed, model, head, device, layers):
    for layer in layers:
        layer.k_cache.zero_()
        layer.v_cache.zero_()
    seqs = [Seq(p, t) for p, t in zip(prompts, tables)]
    first = _prefill(mixed, model, head, seqs, device)
    for s, t in zip(seqs, first):
        s.token_ids.append(t)
        s.is_prefill = False
        s.num_cached_tokens = len(s.token_ids) - 1
    return seqs


def test_model_greedy_spec_equals_plain(device):
    model = Qwen3Segments(num_layers=LAYERS, device=device, seed=7, max_tokens=1024, row_invariant=True)
    head = LMHeadVerifier(model.lm_head)
    rng = np.random.default_rng(8)
    lens = [5, 23, 70, 130, 256, 300]
    steps = 40
    B = len(lens)
    W = max(math.ceil((L + steps + 2 * K + 2) / BLOCK) for L in lens)
    NB = B * W + 1
    layers = _caches(device, NB)
    perm = rng.permutation(NB)
    tables = [perm[b * W:(b + 1) * W].tolist() for b in range(B)]
    prompts = [rng.integers(0, 151936, size=L).tolist() for L in lens]
    mixed = MixedStepRunner(layers, HQ, HKV, D, D ** -0.5, block_size=BLOCK, max_num_batched_tokens=1024,
                            max_num_seqs=8, table_width=W, segment=model, pre_attn=model.pre_attn())
    dec = DecodeStepRunner(layers, model, HQ, HKV, D, D ** -0.5, BLOCK, table_width=W, max_batch=16,
                           query_tokens=(1, 1 + K))
    zeros = torch.zeros(B, device=device)

    seqs = _start(prompts, tables, mixed, model, head, device, layers)
    for _ in range(steps + 2 * K):
        h = dec.run(dec.prepare(seqs, 1, with_drafts=False))
        for s, t in zip(seqs, lm_head_sample(h, head, zeros).tolist()):
            s.token_ids.append(t)
    plain = [s.token_ids for s in seqs]

    seqs = _start(prompts, tables, mixed, model, head, device, layers)
    assert [s.token_ids for s in seqs] == [p[:len(s.token_ids)] for p, s in zip(plain, seqs)]
    accepted = []
    while min(len(s.token_ids) - L for s, L in zip(seqs, lens)) < steps + 1:
        for s, ref in zip(seqs, plain):
            n = len(s.token_ids)
            d = [ref[n + i] if n + i < len(ref) else 0 for i in range(K)]
            s.draft_token_ids = [int(rng.integers(0, 151936)) if rng.random() < 0.3 else x for x in d]
        h = dec.run(dec.prepare(seqs, 1 + K))
        drafts = torch.tensor([s.draft_token_ids for s in seqs], dtype=torch.int64, device=device)
        nd = torch.full((B,), K, dtype=torch.int64, device=device)
        acc, nxt = lm_head_verify(h, head, drafts, nd, zeros)
        for s, a, t in zip(seqs, acc.tolist(), nxt.tolist()):
            s.token_ids += s.draft_token_ids[:a] + [t]
            accepted.append(a)
    print(f"accepted per verify step: {np.bincount(accepted, minlength=K + 1).tolist()}; "
          f"distinct plain tokens {len(set(t for p, L in zip(plain, lens) for t in p[L:]))}", flush=True)
    assert 0 in accepted and K in accepted
    for L, a, b in zip(lens, plain, [s.token_ids for s in seqs]):
        n = L + steps + 1
        assert a[:n] == b[:n], f"spec tokens differ from plain tokens: {a[L:n]} vs {b[L:n]}"
