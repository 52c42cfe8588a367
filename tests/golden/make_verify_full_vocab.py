"""Writes tests/golden/verify_full_vocab.npz: outputs of the reference verifier at the full Qwen3 vocabulary.

The inputs (64 sequences x 4 guess slots x 151,936 tokens, temperatures 0 / 0.05 / 0.1 / 0.5-2, fp32 and bf16
logits, n-gram and draft-model guesses, ragged num_drafts, -inf masks) are regenerated from seeds by
tests/golden/verify_inputs.py, so the fixture keeps only each case's name, its input checksum and the
reference's (num_accepted, next_token). The reference's own nanovllm/layers/sampler.py is loaded on its own
from /root/reference on the CPU, with its two internal random draws replaced by the case's uniforms and
noise (as make_verify_vectors.py does). Only this container has /root/reference.

    python tests/golden/make_verify_full_vocab.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import verify_inputs  # noqa: E402
from make_verify_vectors import load_reference, run_reference  # noqa: E402

OUT = os.path.join(HERE, "verify_full_vocab.npz")


def main():
    ref = load_reference()
    arrays = {}
    for name in verify_inputs.CASES:
        logits, drafts, nd, temps, dl, u, e = verify_inputs.make_case(name)
        a, t = run_reference(ref, logits, drafts, nd, temps, dl, u, e)
        arrays[f"{name}.num_accepted"] = a.numpy().astype(np.int64)
        arrays[f"{name}.next_token"] = t.numpy().astype(np.int64)
        arrays[f"{name}.checksum"] = np.array(verify_inputs.checksum((logits, drafts, nd, temps, dl, u, e)))
        print(f"{name}: accepted {a.tolist()[:16]}... next {t.tolist()[:8]}...", flush=True)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
