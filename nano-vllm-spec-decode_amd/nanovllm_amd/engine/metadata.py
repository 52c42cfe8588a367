"""Host-side builders of the attention metadata a model runner puts in the Context.

They reproduce the batch layouts of the reference runner (nanovllm/engine/model_runner.py):
  * ``mixed_batch``       model_runner.py:31-63  (one flat varlen batch of decode rows then prefill chunks)
  * ``decode_batch``      model_runner.py:319-362 (every sequence brings n query tokens; the batch is padded
                          to a graph bucket with empty sequences: slot -1, context length 0)
  * ``pad_block_tables``  model_runner.py:269-274 (-1 padded rows, optionally to a fixed width)
  * ``batch_buckets``     model_runner.py:26-28
Sequences are duck-typed like the reference's Sequence: ``token_ids`` (indexable), ``last_token``,
``num_tokens`` / ``len()``, ``num_cached_tokens``, ``num_scheduled_tokens``, ``is_prefill``,
``block_table`` and ``draft_token_ids``.
"""


def batch_buckets(max_bs: int) -> list[int]:
    """Batch sizes graphs are recorded for: 1, 2, 4, 8 (below max_bs), multiples of 16, then max_bs."""
    small = [b for b in (1, 2, 4, 8) if b < max_bs]
    return small + list(range(16, max_bs, 16)) + [max_bs]


def _slot(block_table, pos: int, block_size: int) -> int:
    return block_table[pos // block_size] * block_size + pos % block_size


def _num_tokens(seq) -> int:
    return seq.num_tokens if hasattr(seq, "num_tokens") else len(seq)


def mixed_batch(seqs, k: int, block_size: int) -> dict:
    """Flat layout of a mixed step: for each request in order, its query rows (a decode request: the last
    token plus k guess slots, padded by repeating the last one; a prefill request: its scheduled chunk),
    their positions and cache slots; cu_seqlens_k counts every key up to the end of the request's rows;
    logits_indices lists all 1+k rows of a decode request and the last row of a prefill request's final chunk."""
    input_ids, positions, slot_mapping, logits_indices = [], [], [], []
    cu_q, cu_k = [0], [0]
    for seq in seqs:
        if seq.is_prefill:
            first = seq.num_cached_tokens
            last = first + seq.num_scheduled_tokens
            ids = list(seq.token_ids[first:last])
        else:
            first = _num_tokens(seq) - 1
            last = first + 1 + k
            ids = [seq.last_token] + list(seq.draft_token_ids)
            ids += [ids[-1]] * (1 + k - len(ids))
        row0 = cu_q[-1]
        input_ids += ids
        positions += list(range(first, last))
        slot_mapping += [_slot(seq.block_table, pos, block_size) for pos in range(first, last)]
        cu_q.append(row0 + last - first)
        cu_k.append(cu_k[-1] + last)
        if not seq.is_prefill:
            logits_indices += list(range(row0, row0 + 1 + k))
        elif last == _num_tokens(seq):
            logits_indices.append(row0 + last - first - 1)
    lens_q = [b - a for a, b in zip(cu_q, cu_q[1:])]
    lens_k = [b - a for a, b in zip(cu_k, cu_k[1:])]
    return dict(input_ids=input_ids, positions=positions, slot_mapping=slot_mapping, logits_indices=logits_indices,
                cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=max(lens_q), max_seqlen_k=max(lens_k))


def pad_block_tables(seqs, num_padding_seqs: int = 0, width: int = 0) -> list[list[int]]:
    """Block tables as rows of equal width (at least `width`), -1 padded, plus all -1 rows for padding sequences."""
    w = max([width] + [len(seq.block_table) for seq in seqs])
    rows = [list(seq.block_table) + [-1] * (w - len(seq.block_table)) for seq in seqs]
    return rows + [[-1] * w for _ in range(num_padding_seqs)]


def decode_batch(seqs, num_query_tokens: int, block_size: int, buckets: list[int] | None = None,
                 table_width: int = 0, with_drafts: bool = True, num_last_tokens: int = 1) -> dict:
    """Decode / verify step layout: each sequence feeds its last num_last_tokens tokens, then (with_drafts) its
    guesses, padded to num_query_tokens by repeating the last token; context_lens count the cache up to the
    end of those rows. With `buckets` the batch is padded to the next bucket with empty sequences
    (token 0, position 0, slot -1, context length 0). Block tables are padded to `table_width`."""
    input_ids, positions, slot_mapping, context_lens = [], [], [], []
    n = num_query_tokens
    for seq in seqs:
        if num_last_tokens == 1:
            ids = [seq.last_token]
        else:
            ids = list(seq.token_ids[_num_tokens(seq) - num_last_tokens:_num_tokens(seq)])
        if with_drafts:
            ids += list(seq.draft_token_ids)
        ids += [ids[-1]] * (n - len(ids))
        first = _num_tokens(seq) - num_last_tokens
        input_ids += ids
        positions += list(range(first, first + n))
        context_lens.append(first + n)
        slot_mapping += [_slot(seq.block_table, pos, block_size) for pos in range(first, first + n)]
    pad = 0
    if buckets and len(seqs) <= buckets[-1]:
        pad = next(b for b in buckets if b >= len(seqs)) - len(seqs)
        input_ids += [0] * (pad * n)
        positions += [0] * (pad * n)
        slot_mapping += [-1] * (pad * n)
        context_lens += [0] * pad
    return dict(input_ids=input_ids, positions=positions, slot_mapping=slot_mapping, context_lens=context_lens,
                block_tables=pad_block_tables(seqs, pad, table_width), num_padding=pad)
