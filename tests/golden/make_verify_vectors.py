"""Writes tests/golden/verify_vectors.npz: input/output vectors of the reference verifier.

Runs the reference's own nanovllm/layers/sampler.py (loaded on its own from /root/reference, on the CPU;
it imports only torch) on seeded inputs. Its two internal random draws, torch.rand(S, K) and
exponential_(1) on an [S, V] tensor, are replaced for the duration of the call by tensors stored in the
fixture, so any implementation given the same uniforms / noise must return the same accepted counts and
tokens. The reference is only read where this script runs; the tests read the .npz alone.

    python tests/golden/make_verify_vectors.py
"""
import importlib.util
import os

import numpy as np
import torch

REF = "/root/reference/nanovllm/layers/sampler.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "verify_vectors.npz")


def load_reference():
    spec = importlib.util.spec_from_file_location("reference_sampler", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def run_reference(ref, logits, drafts, num_drafts, temps, draft_logits, uniforms, noise):
    rand, exponential = torch.rand, torch.Tensor.exponential_
    try:
        torch.rand = lambda *a, **kw: uniforms.clone()
        torch.Tensor.exponential_ = lambda self, *a, **kw: self.copy_(noise)
        a, t = ref.verify_drafts(logits, drafts, num_drafts, temps, draft_logits)
    finally:
        torch.rand, torch.Tensor.exponential_ = rand, exponential
    return a, t


def make_case(gen, S, K, V, temps, dtype, with_draft, force_reject=False, self_draft=False):
    logits = torch.randn(S * (K + 1), V, generator=gen) * 3
    draft_logits = None
    if with_draft:
        draft_logits = (logits.view(S, K + 1, V)[:, :K] + torch.randn(S, K, V, generator=gen)).contiguous()
        if self_draft:
            draft_logits = logits.view(S, K + 1, V)[:, :K].clone()
        t = torch.where(temps == 0, 1.0, temps)
        probs = torch.softmax(draft_logits / t[:, None, None], -1)
        drafts = torch.multinomial(probs.view(-1, V), 1, generator=gen).view(S, K)
    else:
        top = logits.view(S, K + 1, V).argmax(-1)[:, :K]
        other = torch.randint(0, V, (S, K), generator=gen)
        drafts = torch.where(torch.rand(S, K, generator=gen) < 0.7, top, other)
    # 5% of target rows get the draft's argmax planted (config-4 style agreement)
    plant = torch.rand(S, K, generator=gen) < 0.05
    lv = logits.view(S, K + 1, V)
    for s, j in plant.nonzero().tolist():
        lv[s, j, drafts[s, j]] = lv[s, j].max() + 1.0
    num_drafts = torch.randint(0, K + 1, (S,), generator=gen)
    num_drafts[0] = K
    uniforms = torch.ones(S, K) if force_reject else torch.rand(S, K, generator=gen)
    noise = torch.empty(S, V).exponential_(1, generator=gen)
    logits = logits.to(dtype)
    if draft_logits is not None:
        draft_logits = draft_logits.to(dtype)
    return logits, drafts, num_drafts, temps, draft_logits, uniforms, noise


def to_np(x):
    if x is None:
        return np.zeros(0, np.float32)
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).numpy().view(np.uint16)
    return x.numpy()


def main():
    ref = load_reference()
    gen = torch.Generator().manual_seed(1234)
    S, K, V = 8, 4, 512
    cases = {
        "greedy_f32": dict(temps=torch.zeros(S), dtype=torch.float32, with_draft=False),
        "ngram_t1_f32": dict(temps=torch.ones(S), dtype=torch.float32, with_draft=False),
        "draft_t07_f32": dict(temps=torch.full((S,), 0.7), dtype=torch.float32, with_draft=True),
        "mixed_temps_bf16": dict(temps=torch.tensor([0, 1, 0.5, 0, 1.3, 0, 1, 0.8]), dtype=torch.bfloat16,
                                 with_draft=True),
        "ngram_mixed_bf16": dict(temps=torch.tensor([1, 0, 1, 0.6, 0, 1, 2.0, 0]), dtype=torch.bfloat16,
                                 with_draft=False),
        "zero_residual_f32": dict(temps=torch.ones(S), dtype=torch.float32, with_draft=True, force_reject=True,
                                  self_draft=True),
    }
    arrays = {}
    for name, kw in cases.items():
        logits, drafts, nd, temps, dl, u, e = make_case(gen, S, K, V, **kw)
        if name == "zero_residual_f32":
            logits.view(S, K + 1, V)[..., 0] = -float("inf")   # token 0 impossible (reference unit test idea)
            dl = logits.view(S, K + 1, V)[:, :K].clone()
        a, t = run_reference(ref, logits, drafts, nd, temps, dl, u, e)
        for key, val in dict(logits=logits, drafts=drafts, num_drafts=nd, temps=temps, draft_logits=dl, uniforms=u,
                             noise=e, num_accepted=a, next_token=t).items():
            arrays[f"{name}.{key}"] = to_np(val)
        arrays[f"{name}.dtype"] = np.array(0 if logits.dtype == torch.bfloat16 else 1)
        print(f"{name}: accepted {a.tolist()} next {t.tolist()}")
    # K = 0 (no guesses): plain sampling / greedy
    logits = torch.randn(4, V, generator=gen) * 3
    temps = torch.tensor([0.0, 1.0, 0.5, 0.0])
    e = torch.empty(4, V).exponential_(1, generator=gen)
    drafts = torch.zeros(4, 0, dtype=torch.int64)
    nd = torch.zeros(4, dtype=torch.int64)
    a, t = run_reference(ref, logits, drafts, nd, temps, None, torch.zeros(4, 0), e)
    for key, val in dict(logits=logits, drafts=drafts, num_drafts=nd, temps=temps, draft_logits=None,
                         uniforms=torch.zeros(4, 0), noise=e, num_accepted=a, next_token=t).items():
        arrays[f"k0_sample_f32.{key}"] = to_np(val)
    arrays["k0_sample_f32.dtype"] = np.array(1)
    print(f"k0_sample_f32: next {t.tolist()}")
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
