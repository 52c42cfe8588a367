"""Oracle for the speculative-decoding verifier and the token sampler. Test infrastructure only.

Restates nanovllm/layers/sampler.py on the CPU with the same sequence of
PyTorch fp32 operations, so that its bits follow the reference's. The only
change is the randomness: the reference draws u = torch.rand(S, K)
(sampler.py:77) and E = exponential_(1) [S, V] (sampler.py:101, and :15 in
Sampler.forward) internally; here both are arguments (``uniforms`` and
``exp_noise``), so a GPU implementation given the same tensors must produce
the same accepted counts and tokens.
"""
import torch


def chunked_logsumexp(logits: torch.Tensor, temps: torch.Tensor, chunk_rows: int = 256) -> torch.Tensor:
    """logsumexp(logits[i] / temps[i]) per row in fp32, 256 rows at a time (sampler.py:19-25)."""
    out = torch.empty(logits.size(0), dtype=torch.float32)
    for i in range(0, logits.size(0), chunk_rows):
        rows = logits[i:i + chunk_rows].float() / temps[i:i + chunk_rows, None]
        out[i:i + chunk_rows] = torch.logsumexp(rows, dim=-1)
    return out


def verify_drafts(logits: torch.Tensor, draft_token_ids: torch.Tensor, num_drafts: torch.Tensor,
                  temperatures: torch.Tensor, draft_logits: torch.Tensor | None = None,
                  uniforms: torch.Tensor | None = None, exp_noise: torch.Tensor | None = None):
    """(num_accepted [S] int64, next_token [S] int64) for logits [S*(K+1), V] (sampler.py:28-103).

    uniforms [S, K] fp32 and exp_noise [S, V] fp32 replace the reference's internal torch.rand / exponential_;
    they are only read when some temperature is non-zero, as in the reference."""
    S, K = draft_token_ids.shape
    V = logits.size(-1)
    logits = logits.view(S, K + 1, V)
    rows = torch.arange(S)
    greedy = temperatures == 0
    temps = torch.where(greedy, 1.0, temperatures).float()         # sampler.py:63
    any_random = not bool(greedy.all())                              # sampler.py:64

    top1 = logits.argmax(dim=-1)                                     # sampler.py:66, first index on ties
    accepted = top1[:, :K] == draft_token_ids
    if any_random and K > 0:
        def draft_probability(table):                                # sampler.py:70-74
            lse = chunked_logsumexp(table.reshape(-1, V), temps.repeat_interleave(table.size(1)))
            lse = lse.view(S, table.size(1))[:, :K]
            chosen = table[:, :K].gather(-1, draft_token_ids.unsqueeze(-1)).squeeze(-1).float()
            return torch.exp(chosen / temps[:, None] - lse)
        p_guess = draft_probability(logits)
        q_guess = torch.ones_like(p_guess) if draft_logits is None else draft_probability(draft_logits)
        u = uniforms.float()
        accepted = torch.where(greedy[:, None], accepted, u * q_guess < p_guess)   # sampler.py:78
    accepted &= torch.arange(K) < num_drafts.unsqueeze(1)            # sampler.py:79
    num_accepted = accepted.int().cumprod(dim=1).sum(dim=1)          # sampler.py:80: unbroken leading run

    next_token = top1[rows, num_accepted]
    if any_random:
        p = torch.softmax(logits[rows, num_accepted].float() / temps[:, None], dim=-1)   # sampler.py:84
        if K > 0:
            rejected = num_accepted < num_drafts
            j = num_accepted.clamp(max=K - 1)
            if draft_logits is None:                                 # sampler.py:88-91 (n-gram: q one-hot)
                d = draft_token_ids[rows, j].unsqueeze(1)
                p.scatter_(1, d, torch.where(rejected[:, None], 0.0, p.gather(1, d)))
            else:                                                    # sampler.py:93-99
                q = torch.softmax(draft_logits[rows, j].float() / temps[:, None], dim=-1)
                residual = (p - q).clamp_min_(0)
                rejected &= residual.sum(dim=-1) > 0                 # all-zero residual guard (:98)
                p = torch.where(rejected[:, None], residual, p)
        noise = exp_noise.float()
        sampled = p.div_(noise.clamp_min(1e-10)).argmax(dim=-1)     # sampler.py:101
        next_token = torch.where(greedy, next_token, sampled)
    return num_accepted.to(torch.int64), next_token.to(torch.int64)


def sample(logits: torch.Tensor, temperatures: torch.Tensor, exp_noise: torch.Tensor) -> torch.Tensor:
    """Sampler.forward (sampler.py:5-16) with injected Exp(1) noise [S, V]: greedy argmax where T == 0,
    else argmax(softmax(logits / T) / max(E, 1e-10))."""
    logits = logits.float()
    greedy_tokens = logits.argmax(dim=-1)
    greedy = temperatures == 0
    logits = logits / torch.where(greedy, 1.0, temperatures).unsqueeze(dim=1)
    probs = torch.softmax(logits, dim=-1)
    sampled = probs.div_(exp_noise.float().clamp_min(1e-10)).argmax(dim=-1)
    return torch.where(greedy, greedy_tokens, sampled)
