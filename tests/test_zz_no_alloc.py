"""The allocation-free verifier entry point (sd_verify_drafts_noalloc, scratch in a static device array)
against the workspace entry point (sd_verify_drafts) through the C ABI: identical accepted counts and tokens on
two calls in a row, the second with a smaller input (the scratch keeps the first call's contents), plus a
greedy-only call and the size limit."""
import ctypes

import pytest
import torch

from nanovllm_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(seed, S, K, V, draft, dtype, temps):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(S * (K + 1), V, generator=g) * 3).to(dtype)
    dl = (torch.randn(S * K, V, generator=g) * 3).to(dtype) if draft else None
    drafts = torch.randint(0, V, (S, K), generator=g)
    top = logits.float().view(S, K + 1, V)[:, :K].argmax(-1)
    drafts = torch.where(torch.rand(S, K, generator=g) < 0.5, top, drafts)
    nd = torch.randint(0, K + 1, (S,), generator=g)
    t = torch.tensor(temps, dtype=torch.float32).repeat(S // len(temps) + 1)[:S]
    u = torch.rand(S, K, generator=g)
    e = torch.empty(S, V).exponential_(1, generator=g)
    return logits, dl, drafts, nd, t, u, e


def _call(lib, noalloc, device, logits, dl, drafts, nd, temps, u, e, greedy_only=False):
    S, K = drafts.shape
    V = logits.size(-1)
    dt = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}
    x = [t.to(device).contiguous() if t is not None else None for t in (logits, dl, drafts, nd, temps, u, e)]
    logits, dl, drafts, nd, temps, u, e = x
    acc = torch.full((S,), -7, dtype=torch.int64, device=device)
    nxt = torch.full((S,), -7, dtype=torch.int64, device=device)
    tp = None if greedy_only else temps.data_ptr()
    args = [logits.data_ptr(), dt[logits.dtype], V, drafts.data_ptr(), nd.data_ptr(), tp, _lib.ptr(dl),
            dt[dl.dtype] if dl is not None else 0, V if dl is not None else 0, None if greedy_only else u.data_ptr(),
            None if greedy_only else e.data_ptr(), S, K, V, acc.data_ptr(), nxt.data_ptr()]
    stream = _lib.stream_of(device)
    if noalloc:
        rc = lib.sd_verify_drafts_noalloc(*args, stream)
    else:
        ws = torch.empty(lib.sd_verify_workspace_size(S, K, V, int(dl is not None)), dtype=torch.uint8, device=device)
        rc = lib.sd_verify_drafts(*args, ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return acc.cpu(), nxt.cpu()


def test_noalloc_matches_workspace_entry_point(device):
    lib = _lib.load()
    cases = [  # a large call, then a smaller one that reuses the scratch the first left behind
        (_inputs(1, 64, 4, 151936, True, torch.float32, [0.0, 1.0, 0.7, 0.1]), False),
        (_inputs(2, 8, 2, 50000, False, torch.bfloat16, [1.0, 0.0, 0.5]), False),
        (_inputs(3, 16, 3, 151936, True, torch.bfloat16, [0.0]), True),            # greedy only: temps NULL
    ]
    for i, (inp, greedy_only) in enumerate(cases):
        print(f"case {i}: S={inp[2].size(0)} K={inp[2].size(1)} V={inp[0].size(-1)} greedy_only={greedy_only}",
              flush=True)
        a0, t0 = _call(lib, False, device, *inp, greedy_only=greedy_only)
        a1, t1 = _call(lib, True, device, *inp, greedy_only=greedy_only)
        assert a1.tolist() == a0.tolist() and t1.tolist() == t0.tolist(), i
        assert (a1 >= 0).all() and (t1 >= 0).all()


def test_noalloc_rejects_sizes_beyond_its_scratch(device):
    lib = _lib.load()
    S, K, V = 4096, 15, 151936
    assert lib.sd_verify_workspace_size(S, K, V, 1) > 8 << 20
    dummy = torch.zeros(16, dtype=torch.int64, device=device)
    p = dummy.data_ptr()
    rc = lib.sd_verify_drafts_noalloc(p, _lib.DTYPE_F32, V, p, p, p, p, _lib.DTYPE_F32, V, p, p, S, K, V, p, p,
                                      _lib.stream_of(device))
    assert rc == 2 and b"scratch" in lib.sd_last_error()
    assert ctypes.c_int(rc).value == 2


_CAPTURE_SCRIPT = r"""
import sys, torch
sys.path[:0] = {paths!r}
from nanovllm_amd import _lib
dev = torch.device("cuda:0")
lib = _lib.load()
g = torch.Generator().manual_seed(5)
S, K, V = 32, 4, 151936
logits = (torch.randn(S * (K + 1), V, generator=g) * 3).to(dev)
drafts = logits.view(S, K + 1, V)[:, :K].argmax(-1).contiguous()
drafts[::3, 1] = 7
nd = torch.full((S,), K, dtype=torch.int64, device=dev)
temps = torch.tensor([0.0, 1.0] * (S // 2), device=dev)
u = torch.rand(S, K, generator=g).to(dev)
e = torch.empty(S, V).exponential_(1, generator=g).to(dev)
acc = torch.empty(S, dtype=torch.int64, device=dev)
nxt = torch.empty(S, dtype=torch.int64, device=dev)
def call(fn, *ws):
    return fn(logits.data_ptr(), _lib.DTYPE_F32, V, drafts.data_ptr(), nd.data_ptr(), temps.data_ptr(), None, 0, 0,
              u.data_ptr(), e.data_ptr(), S, K, V, acc.data_ptr(), nxt.data_ptr(), *ws,
              torch.cuda.current_stream().cuda_stream)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = call(lib.sd_verify_drafts_noalloc)       # the library's first call on this device, under capture
_lib.check(rc, "sd_verify_drafts_noalloc")
ws = torch.empty(lib.sd_verify_workspace_size(S, K, V, 0), dtype=torch.uint8, device=dev)
_lib.check(call(lib.sd_verify_drafts, ws.data_ptr(), ws.numel()), "sd_verify_drafts")
ref = (acc.cpu().clone(), nxt.cpu().clone())
for rep in range(3):
    acc.fill_(-5)
    nxt.fill_(-5)
    graph.replay()
    torch.cuda.synchronize()
    assert acc.cpu().tolist() == ref[0].tolist() and nxt.cpu().tolist() == ref[1].tolist(), rep
    torch.randn(1000, device=dev).sum().item()     # the program's own eager work between replays
print("capture ok", ref[0].tolist()[:8])
"""


def test_noalloc_first_call_under_graph_capture(device):
    """The entry point's first call on a device happens while a HIP graph is being captured (a fresh process):
    the scratch address is looked up then, the call is recorded, and three replays, with eager work between
    them, give what the workspace entry point gives."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    paths = [root, os.path.join(root, "nano-vllm-spec-decode_amd")]
    res = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT.format(paths=paths)], capture_output=True, text=True,
                         timeout=240)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "capture ok" in res.stdout
