"""Host-side batch layout builders (CPU): the reference's mixed_batch known answer
(tests/test_spec_unit.py:682-699, block size 4) and the decode / verify padding rules of
nanovllm/engine/model_runner.py:319-362."""
from types import SimpleNamespace

from nanovllm_amd.engine.metadata import batch_buckets, decode_batch, mixed_batch, pad_block_tables

BS = 4


def seq(tokens, **kw):
    s = SimpleNamespace(token_ids=list(tokens), last_token=tokens[-1], num_tokens=len(tokens), num_cached_tokens=0,
                        num_scheduled_tokens=0, is_prefill=True, block_table=[], draft_token_ids=[])
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_mixed_batch_known_answer():
    dec = seq([1, 2, 3, 4, 5, 6], is_prefill=False, num_cached_tokens=5, block_table=[7, 3], draft_token_ids=[9])
    first = seq(list(range(10, 20)), num_scheduled_tokens=6, block_table=[0, 1, 2])
    last = seq(list(range(20, 25)), num_cached_tokens=4, num_scheduled_tokens=1, block_table=[4, 5])
    b = mixed_batch([dec, first, last], 2, BS)
    assert b["input_ids"] == [6, 9, 9] + list(range(10, 16)) + [24]
    assert b["positions"] == [5, 6, 7] + list(range(6)) + [4]
    assert b["slot_mapping"] == [3 * BS + 1, 3 * BS + 2, 3 * BS + 3] + [0, 1, 2, 3, 4, 5] + [5 * BS]
    assert b["cu_seqlens_q"] == [0, 3, 9, 10] and b["cu_seqlens_k"] == [0, 8, 14, 19]
    assert b["max_seqlen_q"] == 6 and b["max_seqlen_k"] == 8
    assert b["logits_indices"] == [0, 1, 2, 9]


def test_batch_buckets():
    assert batch_buckets(512)[:6] == [1, 2, 4, 8, 16, 32] and batch_buckets(512)[-1] == 512
    assert batch_buckets(102) == [1, 2, 4, 8, 16, 32, 48, 64, 80, 96, 102]
    assert batch_buckets(3) == [1, 2, 3]


def test_decode_batch_verify_padding():
    a = seq(list(range(9)), block_table=[2, 5, 6], draft_token_ids=[50, 51])
    b = seq(list(range(4)), block_table=[1, 9], draft_token_ids=[])
    d = decode_batch([a, b], 4, BS, buckets=[1, 4, 8], table_width=3)
    # each sequence: last token, its guesses, then the last one repeated up to 1 + k = 4 rows
    assert d["input_ids"] == [8, 50, 51, 51, 3, 3, 3, 3] + [0] * 8
    assert d["positions"] == [8, 9, 10, 11, 3, 4, 5, 6] + [0] * 8
    slot = lambda table, p: table[p // BS] * BS + p % BS       # model_runner.py:338
    assert d["slot_mapping"] == [slot([2, 5, 6], p) for p in range(8, 12)] + [slot([1, 9], p) for p in range(3, 7)] \
        + [-1] * 8
    assert d["slot_mapping"][:8] == [6 * BS, 6 * BS + 1, 6 * BS + 2, 6 * BS + 3, 1 * BS + 3, 9 * BS, 9 * BS + 1, 9 * BS + 2]
    assert d["context_lens"] == [12, 7, 0, 0]
    assert d["block_tables"] == [[2, 5, 6], [1, 9, -1], [-1, -1, -1], [-1, -1, -1]]
    assert d["num_padding"] == 2


def test_pad_block_tables_width():
    a, b = seq([1], block_table=[3]), seq([1], block_table=[4, 5])
    assert pad_block_tables([a, b], 1, 4) == [[3, -1, -1, -1], [4, 5, -1, -1], [-1, -1, -1, -1]]
