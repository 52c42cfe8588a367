"""Host side of the mixed-step graph runtime (CPU): bucket lists and the padded metadata layout a graph
replays with (one padding sequence holding the padding rows with no keys, empty sequences after it, -1
slots and -1 block-table rows)."""
from types import SimpleNamespace

import pytest

from nanovllm_amd.engine.mixed_step import mixed_step_layout, seq_buckets, token_buckets

BS = 4


def seq(tokens, **kw):
    s = SimpleNamespace(token_ids=list(tokens), last_token=tokens[-1], num_tokens=len(tokens), num_cached_tokens=0,
                        num_scheduled_tokens=0, is_prefill=True, block_table=[], draft_token_ids=[])
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_buckets():
    assert token_buckets(2048)[:3] == [16, 32, 48] and token_buckets(2048)[-1] == 2048
    assert len(token_buckets(2048)) == 128
    assert token_buckets(2048, 64)[:3] == [64, 128, 192] and len(token_buckets(2048, 64)) == 32
    assert token_buckets(100, 64) == [64, 100]
    assert seq_buckets(256) == [2, 4] + list(range(8, 257, 8)) + [257]
    assert seq_buckets(64) == [2, 4, 8, 16, 24, 32, 40, 48, 56, 64, 65]
    assert seq_buckets(63) == [2, 4, 8, 16, 24, 32, 40, 48, 56, 64]
    assert seq_buckets(7) == [2, 4, 8] and seq_buckets(3) == [2, 4] and seq_buckets(1) == [2]
    assert seq_buckets(256, 64) == [2, 4, 64, 128, 192, 256, 257]


def test_padded_layout_known_answer():
    dec = seq([1, 2, 3, 4, 5, 6], is_prefill=False, num_cached_tokens=5, block_table=[7, 3], draft_token_ids=[9])
    first = seq(list(range(10, 20)), num_scheduled_tokens=6, block_table=[0, 1, 2])
    W = 4
    b = mixed_step_layout([dec, first], 2, BS, W, [8, 16], [2, 4, 8])
    n, N, S = b["n"], b["N"], b["S"]
    assert (n, N, S) == (9, 16, 4)
    meta = b["meta"]
    cu_q, cu_k = meta[:S + 1], meta[S + 1:2 * (S + 1)]
    slots, tables = meta[2 * (S + 1):2 * (S + 1) + N], meta[2 * (S + 1) + N:]
    assert cu_q == [0, 3, 9, 16, 16]            # decode 1+k rows, prefill chunk 6, padding rows 9..15, empty
    assert cu_k == [0, 8, 14, 14, 14]           # padding sequences see no keys
    assert slots == [3 * BS + 1, 3 * BS + 2, 3 * BS + 3, 0, 1, 2, 3, 4, 5] + [-1] * 7
    assert tables == [7, 3, -1, -1, 0, 1, 2, -1] + [-1] * 8
    assert len(meta) == 2 * (S + 1) + N + S * W
    assert b["positions_padded"] == [5, 6, 7, 0, 1, 2, 3, 4, 5] + [0] * 7   # padding rows at position 0


def test_layout_limits():
    long = seq(list(range(20)), num_scheduled_tokens=20, block_table=[0, 1, 2, 3, 4])
    with pytest.raises(ValueError, match="width"):
        mixed_step_layout([long], 0, BS, 4, [64], [2])
    with pytest.raises(ValueError, match="largest bucket"):
        mixed_step_layout([long], 0, BS, 8, [16], [2])
