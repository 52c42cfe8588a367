"""Oracle for the paged KV-cache scatter. Test infrastructure only.

Follows nanovllm/layers/attention.py:10-40 (store_kvcache_kernel + store_kvcache):
for every token row idx with slot_mapping[idx] != -1, row idx of key / value
(Hkv*D contiguous elements, arbitrary row stride) is copied into slot
slot_mapping[idx] of the caches viewed as [NB*block_size, Hkv*D].
A pure copy, so the GPU result must match bit for bit.
"""
import torch


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """In-place scatter into k_cache / v_cache ([NB, bs, Hkv, D]); -1 slots are skipped (attention.py:23)."""
    N, H, D = key.shape
    assert value.shape == key.shape and slot_mapping.numel() == N
    kc = k_cache.view(-1, H * D)
    vc = v_cache.view(-1, H * D)
    slots = slot_mapping.to(torch.int64).cpu()
    keep = slots != -1
    rows = torch.nonzero(keep).flatten()
    kc.index_copy_(0, slots[keep], key.reshape(N, H * D)[rows])
    vc.index_copy_(0, slots[keep], value.reshape(N, H * D)[rows])
