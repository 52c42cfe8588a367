"""Greedy speculative decoding is token-identical to greedy non-speculative decoding (the property the
reference checks end to end in tests/test_greedy.py on a real model).

A small random model runs through the drop-in pieces: Attention.forward reading the global Context (varlen
prefill of the prompts, then paged decode with one query per sequence, or spec-verify with k+1 queries),
Sampler for the plain steps and verify_drafts (greedy) for the spec steps. Everything outside attention is
computed row by row in float64 on the CPU, so any difference in tokens would come from the attention or
the sampler. Drafts are the plain run's own tokens with some replaced by wrong ones, so that steps accept
everything, nothing, and runs in between."""
import math

import numpy as np
import pytest
import torch

from nanovllm_amd.layers.attention import Attention
from nanovllm_amd.layers.sampler import Sampler, verify_drafts
from nanovllm_amd.utils.context import reset_context, set_context

pytestmark = pytest.mark.gpu

HQ, HKV, D, HID, VOCAB, LAYERS, BLOCK = 8, 2, 128, 256, 512, 2, 256


class TinyModel:
    """Embedding + learned positions, LAYERS x (q/k/v projections -> attention -> output projection, residual),
    tied LM head. Projections in float64 on the CPU, one row at a time."""

    def __init__(self, device, seed=0, max_pos=512):
        g = np.random.default_rng(seed)
        s = 1 / math.sqrt(HID)
        self.emb = g.normal(0, 1, (VOCAB, HID))
        self.pos = g.normal(0, 0.5, (max_pos, HID))
        self.w = [dict(q=g.normal(0, s, (HID, HQ * D)), k=g.normal(0, s, (HID, HKV * D)),
                       v=g.normal(0, s, (HID, HKV * D)), o=g.normal(0, 1 / math.sqrt(HQ * D), (HQ * D, HID)))
                  for _ in range(LAYERS)]
        self.attn = [Attention(HQ, D, D ** -0.5, HKV) for _ in range(LAYERS)]
        nb = 8
        for a in self.attn:
            a.k_cache = torch.zeros(nb, BLOCK, HKV, D, dtype=torch.bfloat16, device=device)
            a.v_cache = torch.zeros(nb, BLOCK, HKV, D, dtype=torch.bfloat16, device=device)
        self.device = device

    @staticmethod
    def _rows(x, w):
        return np.stack([x[i] @ w for i in range(x.shape[0])])

    def forward(self, tokens, positions):
        """Logits (float32, on the GPU) of the given rows; the Context must describe them."""
        h = self.emb[tokens] + self.pos[positions]
        dev = self.device
        for w, attn in zip(self.w, self.attn):
            q = torch.tensor(self._rows(h, w["q"]), dtype=torch.bfloat16, device=dev).view(-1, HQ, D)
            k = torch.tensor(self._rows(h, w["k"]), dtype=torch.bfloat16, device=dev).view(-1, HKV, D)
            v = torch.tensor(self._rows(h, w["v"]), dtype=torch.bfloat16, device=dev).view(-1, HKV, D)
            o = attn(q, k, v).float().cpu().double().reshape(len(tokens), HQ * D).numpy()
            h = h + self._rows(o, w["o"])
        logits = self._rows(h, self.emb.T)
        return torch.tensor(logits, dtype=torch.float32, device=dev)


def _i32(x, dev):
    return torch.tensor(x, dtype=torch.int32, device=dev)


def _prefill(model, prompts, tables):
    """All prompts in one varlen prefill; returns each prompt's first generated token (greedy)."""
    dev = model.device
    toks, pos, slots, cu = [], [], [], [0]
    for p, t in zip(prompts, tables):
        toks += p
        pos += list(range(len(p)))
        slots += [t[i // BLOCK] * BLOCK + i % BLOCK for i in range(len(p))]
        cu.append(cu[-1] + len(p))
    set_context(True, _i32(cu, dev), _i32(cu, dev), max(map(len, prompts)), max(map(len, prompts)), _i32(slots, dev))
    logits = model.forward(np.array(toks), np.array(pos))
    reset_context()
    last = torch.tensor([c - 1 for c in cu[1:]], device=dev)
    temps = torch.zeros(len(prompts), dtype=torch.float32, device=dev)
    return Sampler()(logits[last], temps).tolist()


def _decode_step(model, seqs, tables, n, drafts=None):
    """One decode step over all sequences with n query rows each (the last token, then n-1 drafts). Returns
    the logits [B*n, V]."""
    dev = model.device
    toks, pos, slots, lens = [], [], [], []
    for b, s in enumerate(seqs):
        row = [s[-1]] + (drafts[b] if drafts else [])
        first = len(s) - 1
        toks += row
        pos += list(range(first, first + n))
        slots += [tables[b][p // BLOCK] * BLOCK + p % BLOCK for p in range(first, first + n)]
        lens.append(first + n)
    W = max(len(t) for t in tables)
    bt = _i32([list(t) + [-1] * (W - len(t)) for t in tables], dev)
    set_context(False, slot_mapping=_i32(slots, dev), context_lens=_i32(lens, dev), block_tables=bt)
    logits = model.forward(np.array(toks), np.array(pos))
    reset_context()
    return logits


def _generate_plain(model, prompts, tables, steps):
    seqs = [list(p) + [t] for p, t in zip(prompts, _prefill(model, prompts, tables))]
    temps = torch.zeros(len(seqs), dtype=torch.float32, device=model.device)
    for _ in range(steps):
        nxt = Sampler()(_decode_step(model, seqs, tables, 1), temps).tolist()
        for s, t in zip(seqs, nxt):
            s.append(t)
    return seqs


def _generate_spec(model, prompts, tables, steps, k, oracle, rng, wrong=0.35):
    seqs = [list(p) + [t] for p, t in zip(prompts, _prefill(model, prompts, tables))]
    B, dev = len(seqs), model.device
    accepted_hist = []
    while min(len(s) - len(p) for s, p in zip(seqs, prompts)) < steps + 1:
        drafts = []
        for s, ref in zip(seqs, oracle):
            d = [ref[len(s) + i] if len(s) + i < len(ref) else 0 for i in range(k)]
            d = [int(rng.integers(0, VOCAB)) if rng.random() < wrong else x for x in d]
            drafts.append(d)
        logits = _decode_step(model, seqs, tables, k + 1, drafts)
        acc, nxt = verify_drafts(logits, torch.tensor(drafts, dtype=torch.int64, device=dev),
                                 torch.full((B,), k, dtype=torch.int64, device=dev),
                                 torch.zeros(B, dtype=torch.float32, device=dev))
        for s, d, a, t in zip(seqs, drafts, acc.tolist(), nxt.tolist()):
            s += d[:a] + [t]
            accepted_hist.append(a)
    return seqs, accepted_hist


@pytest.mark.parametrize("k", [1, 2, 4])
def test_greedy_spec_equals_plain(device, k):
    model = TinyModel(device, seed=k)
    rng = np.random.default_rng(100 + k)
    prompts = [rng.integers(0, VOCAB, size=L).tolist() for L in (5, 23, 70)]
    tables = [[0], [3], [5]]
    steps = 40
    plain = _generate_plain(model, prompts, tables, steps + 2 * k)
    spec, acc = _generate_spec(model, prompts, tables, steps, k, plain, rng)
    print(f"k={k}: accepted per step {np.bincount(acc, minlength=k + 1).tolist()}", flush=True)
    assert 0 in acc and k in acc, "the drafts should give both full and empty acceptances"
    for p, a, b in zip(prompts, plain, spec):
        n = len(p) + steps + 1
        assert a[:n] == b[:n], f"spec tokens differ from plain tokens: {a[len(p):n]} vs {b[len(p):n]}"
