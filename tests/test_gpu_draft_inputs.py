"""Draft-step input building on the GPU (HIP sd_draft_step_inputs) against the oracle: bit-exact.

Covers the loop body of ModelRunner.run_draft (nanovllm/engine/model_runner.py:443-452): padding sequences
(context length 0), block-boundary crossings, S < B token rows, every later step j of k = 8, graph capture
with the inputs rewritten in place between replays, and the position past the block table (slot -1 here,
where the reference's gather would fault).
"""
import pytest
import torch

from nanovllm_amd.engine.draft_inputs import DraftStepBuffers, draft_step_inputs
from oracle import draft_inputs as odi

pytestmark = pytest.mark.gpu


def _batch(seed, B=64, S=50, W=33, bs=256):
    g = torch.Generator().manual_seed(seed)
    real_lens = torch.zeros(B, dtype=torch.int32)
    real_lens[:S] = torch.randint(1, W * bs - 16, (S,), generator=g).to(torch.int32)
    last_pos = (real_lens.long() - 1).clamp_min(0)
    last_pos[S:] = torch.randint(0, 100, (B - S,), generator=g)    # padding rows: ignored
    tables = torch.randperm(4096, generator=g)[:B * W].view(B, W).to(torch.int32)
    tables[S:] = -1
    tokens = torch.randint(0, 151936, (S,), generator=g)
    return real_lens, last_pos, tables, tokens, bs


def _equal(got, want):
    return all(torch.equal(a.cpu(), b) for a, b in zip(got, want))


@pytest.mark.parametrize("seed", [0, 1])
def test_every_step_bitexact(device, seed):
    real_lens, last_pos, tables, tokens, bs = _batch(seed)
    # crossings: positions that land on the first slot of a block at some step
    last_pos[0], real_lens[0] = 255, 256
    last_pos[1], real_lens[1] = 510, 511
    dev = [x.to(device) for x in (real_lens, last_pos, tables, tokens)]
    bufs = DraftStepBuffers(real_lens.numel(), device)
    for j in range(1, 8):
        got = draft_step_inputs(dev[0], dev[1], dev[2], bs, dev[3], j, bufs)
        want = odi.draft_step_inputs(real_lens, last_pos, tables, bs, tokens, j)
        torch.cuda.synchronize()
        assert _equal(got, want), f"step {j}"


def test_all_real_and_no_tokens(device):
    real_lens, last_pos, tables, tokens, bs = _batch(2, B=16, S=16, W=4)
    dev = [x.to(device) for x in (real_lens, last_pos, tables)]
    empty = torch.zeros(0, dtype=torch.int64, device=device)
    got = draft_step_inputs(dev[0], dev[1], dev[2], bs, empty, 1)
    want = odi.draft_step_inputs(real_lens, last_pos, tables, bs, torch.zeros(0, dtype=torch.int64), 1)
    torch.cuda.synchronize()
    assert _equal(got, want)


def test_position_past_table_gives_minus_one(device):
    real_lens = torch.tensor([10, 256], dtype=torch.int32, device=device)
    last_pos = torch.tensor([9, 255], dtype=torch.int64, device=device)
    tables = torch.tensor([[3], [4]], dtype=torch.int32, device=device)     # one block each
    ids, pos, slots, lens = draft_step_inputs(real_lens, last_pos, tables, 256,
                                              torch.tensor([7, 8], device=device), 1)
    torch.cuda.synchronize()
    assert pos.tolist() == [10, 256] and lens.tolist() == [11, 257]
    assert slots.tolist() == [3 * 256 + 10, -1] and ids.tolist() == [7, 8]


def test_graph_capture_replays(device):
    real_lens, last_pos, tables, tokens, bs = _batch(3)
    dev = [x.to(device) for x in (real_lens, last_pos, tables, tokens)]
    bufs = DraftStepBuffers(real_lens.numel(), device)
    draft_step_inputs(dev[0], dev[1], dev[2], bs, dev[3], 2, bufs)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        draft_step_inputs(dev[0], dev[1], dev[2], bs, dev[3], 2, bufs)
    for r in range(3):
        nl, np_, nt, ntok, _ = _batch(10 + r)
        for d, s in zip(dev, (nl, np_, nt, ntok)):
            d.copy_(s)
        graph.replay()
        torch.cuda.synchronize()
        got = (bufs.input_ids, bufs.positions, bufs.slot_mapping, bufs.context_lens)
        assert _equal(got, odi.draft_step_inputs(nl, np_, nt, bs, ntok, 2)), f"replay {r}"
