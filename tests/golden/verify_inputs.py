"""Seeded inputs of the full-vocabulary rejection-sampler cases (64 sequences, 4 guess slots, 151,936 tokens).

Both tests/golden/make_verify_full_vocab.py (which runs the reference's sampler.py on them, in the container
that holds the reference) and the tests (which regenerate them to check the GPU verifier and the oracle
against the stored outputs) build their inputs here, so the fixture holds only seeds, parameters, outputs and
a checksum of the inputs. Everything is drawn with numpy's PCG64 generator (reproducible across machines for
one numpy version); bf16 tables are torch's round-to-nearest-even cast of the fp32 draw.

A case:
  target logits  [S*(K+1), V] ~ N(offset, 3^2); draft logits [S, K, V] ~ N(offset, 3^2) (draft-model cases).
  guesses        the draft row's argmax (greedy rows) or a Gumbel-max sample of softmax(draft / T); 30 % of
                 them are replaced by the target row's argmax so that accept runs of every length occur;
                 5 % of (sequence, slot) pairs get the guess planted as the target row's maximum (+1).
  masks          optional: 30 % of the entries of every fourth row set to -inf, and the first 40,000
                 entries of every seventh row (whole spans of -inf); guesses and planted entries stay finite.
  num_drafts     K, or uniform in [0, K] (ragged; sequence 0 keeps K).
  uniforms       U[0, 1) [S, K] fp32; exp_noise Exp(1) [S, V] fp32.
"""
import hashlib

import numpy as np
import torch

S, K, V = 64, 4, 151936

# name -> parameters; the temperatures are per sequence, cycled over the batch
CASES = {
    "t0_f32_ngram": dict(seed=101, temps=[0.0], dtype="f32", draft=False, ragged=False),
    "t0_bf16_draft_ragged": dict(seed=102, temps=[0.0], dtype="bf16", draft=True, ragged=True),
    "t1_f32_ngram_ragged": dict(seed=103, temps=[1.0], dtype="f32", draft=False, ragged=True),
    "t1_f32_draft": dict(seed=104, temps=[1.0], dtype="f32", draft=True, ragged=False),
    "t1_bf16_draft_ragged": dict(seed=105, temps=[1.0], dtype="bf16", draft=True, ragged=True),
    "t005_f32_draft_masked": dict(seed=106, temps=[0.05], dtype="f32", draft=True, ragged=False, offset=-8.0,
                                  masked=True),
    "t01_bf16_ngram_masked": dict(seed=107, temps=[0.1], dtype="bf16", draft=False, ragged=True, offset=-8.0,
                                  masked=True),
    "mixed_f32_draft_ragged": dict(seed=108, temps=[0.0, 0.05, 0.1, 0.5, 0.7, 1.0, 1.5, 2.0], dtype="f32",
                                   draft=True, ragged=True, offset=-4.0, masked=True),
    "k0_f32_sample": dict(seed=109, temps=[0.0, 1.0, 0.1, 0.7], dtype="f32", draft=False, ragged=False, k=0,
                          masked=True, offset=-6.0),
    "zero_residual_t1_f32": dict(seed=110, temps=[1.0], dtype="f32", draft=True, ragged=False, self_draft=True,
                                 reject_all=True),
}


def _to_torch(x: np.ndarray, dtype: str) -> torch.Tensor:
    t = torch.from_numpy(x)
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def make_case(name: str):
    """(logits [S*(K+1), V], drafts [S, K], num_drafts [S], temps [S], draft_logits [S, K, V] | None,
    uniforms [S, K], exp_noise [S, V]) as CPU tensors, shaped as the reference's verify_drafts takes them."""
    c = CASES[name]
    k = c.get("k", K)
    rng = np.random.default_rng(c["seed"])
    off = np.float32(c.get("offset", 0.0))
    three = np.float32(3.0)
    logits = rng.standard_normal((S, k + 1, V), dtype=np.float32) * three + off
    dlog = rng.standard_normal((S, max(k, 1), V), dtype=np.float32)[:, :k] * three + off
    if c.get("self_draft"):
        dlog = logits[:, :k].copy()
    temps = np.resize(np.asarray(c["temps"], dtype=np.float32), S)
    if c.get("masked"):
        mask_rows = rng.random((S, k + 1)) < 0.25
        logits[mask_rows] = np.where(rng.random((int(mask_rows.sum()), V)) < 0.3, -np.inf, logits[mask_rows])
        logits[::7, :, :40000] = -np.inf
        if k > 0:
            dlog[1::5, :, 100000:140000] = -np.inf
    # guesses: argmax of the draft row, or a Gumbel-max sample of softmax(draft / T)
    drafts = np.zeros((S, k), dtype=np.int64)
    for s in range(S):
        for j in range(k):
            row = dlog[s, j].astype(np.float64)
            if temps[s] == 0:
                drafts[s, j] = int(np.argmax(row))
            else:
                gum = -np.log(-np.log(rng.random(V) * (1 - 1e-12) + 1e-12))
                drafts[s, j] = int(np.argmax(row / float(temps[s]) + gum))
    if k > 0:
        finite_top = np.argmax(logits[:, :k], axis=-1)
        agree = rng.random((S, k)) < 0.3
        drafts = np.where(agree, finite_top, drafts)
        plant = rng.random((S, k)) < 0.05
        for s, j in zip(*np.nonzero(plant)):
            logits[s, j, drafts[s, j]] = np.max(logits[s, j]) + np.float32(1.0)
        for s in range(S):   # a guess under a mask gets a finite target logit back
            for j in range(k):
                d = drafts[s, j]
                if not np.isfinite(logits[s, j, d]):
                    logits[s, j, d] = off
    nd = rng.integers(0, k + 1, size=S) if c["ragged"] else np.full(S, k)
    nd[0] = k
    uniforms = rng.random((S, k), dtype=np.float32)
    if c.get("reject_all"):
        uniforms[:] = np.float32(1.0)
    noise = rng.standard_exponential((S, V), dtype=np.float32)
    draft_logits = _to_torch(np.ascontiguousarray(dlog), c["dtype"]) if c["draft"] else None   # [S, K, V]
    return (_to_torch(np.ascontiguousarray(logits.reshape(S * (k + 1), V)), c["dtype"]), torch.from_numpy(drafts),
            torch.from_numpy(nd.astype(np.int64)), torch.from_numpy(temps), draft_logits,
            torch.from_numpy(uniforms), torch.from_numpy(noise))


def checksum(tensors) -> str:
    """sha256 over the raw bytes of the inputs (None skipped), to detect a regeneration that drifted."""
    h = hashlib.sha256()
    for t in tensors:
        if t is None:
            continue
        t = t.contiguous()
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        h.update(t.numpy().tobytes())
    return h.hexdigest()
