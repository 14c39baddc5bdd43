"""Autoregressive generation with the constant-size recurrent state
(generation.py:23-102 of Chyxx/CyFA-Jittor v0.1.2).

``generate`` continues one prompt (greedy, or temperature / nucleus sampling
from a seeded numpy generator); ``generate_batch`` runs right-padded prompts
through one masked prefill and then greedy decode steps, each row stopping on
its own. Both return token ids as Python lists, as the reference does; the
model runs on whatever device holds its parameters.
"""

import numpy as np
import torch


def _device(model):
    return next(model.parameters()).device


def _nucleus(logits, temperature, top_p, rng):
    """One token from softmax(logits / temperature), restricted to the most
    probable tokens whose preceding cumulative probability is below top_p
    (the smallest set holding top_p of the mass), renormalised."""
    scaled = logits / temperature
    probs = np.exp(scaled - scaled.max())
    probs /= probs.sum()
    order = np.argsort(-probs)
    before = np.cumsum(probs[order]) - probs[order]
    kept = order[before < top_p]
    return int(rng.choice(kept, p=probs[kept] / probs[kept].sum()))


@torch.no_grad()
def generate(model, ids, max_new_tokens=64, eos_token_id=None, temperature=0.0, top_p=1.0, seed=42, on_token=None):
    """New tokens after the prompt ``ids`` (a list of ints). Stops after
    max_new_tokens, on eos_token_id (which is kept), or when
    on_token(generated) returns true. ValueError for an empty prompt, a
    negative length or temperature, or top_p outside (0, 1]."""
    if not ids or max_new_tokens < 0 or temperature < 0 or not 0 < top_p <= 1:
        raise ValueError("Invalid prompt or sampling options")
    model.eval()
    dev = _device(model)
    rng = np.random.default_rng(seed)
    current, cache, generated = list(ids), None, []
    for _ in range(max_new_tokens):
        result = model(torch.tensor([current], dtype=torch.long, device=dev), cache=cache, use_cache=True)
        cache = result["cache"]
        last = result["logits"][0, -1]
        if temperature == 0:
            # greedy: the first largest logit, found on the device (one index
            # crosses to the host, not the row); NaN counts as largest, as in
            # numpy's argmax of the same values
            token = int(last.argmax())
        else:
            token = _nucleus(last.double().cpu().numpy(), temperature, top_p, rng)
        generated.append(token)
        if on_token is not None and on_token(generated):
            break
        if token == eos_token_id:
            break
        current = [token]
    return generated


@torch.no_grad()
def generate_batch(model, prompts, max_new_tokens=48, eos_token_id=None, on_token=None):
    """Greedy continuations of several prompts at once. The prompts are
    right-padded to a multiple of 64 tokens and run through one prefill with
    an attention mask (pads leave the state and the conv cache unchanged);
    each row's first token comes from the logits at its last prompt token.
    A row stops on eos_token_id or when on_token(row_tokens) returns true;
    the loop ends when every row has stopped or after max_new_tokens."""
    if not prompts or any(not ids for ids in prompts) or max_new_tokens < 0:
        raise ValueError("Expected nonempty prompts and a nonnegative generation length")
    model.eval()
    dev = _device(model)
    lengths = torch.tensor([len(ids) for ids in prompts], dtype=torch.long)
    width = int((int(lengths.max()) + 63) // 64 * 64)
    ids = torch.zeros(len(prompts), width, dtype=torch.long)
    mask = torch.zeros_like(ids)
    for row, tokens in enumerate(prompts):
        ids[row, :len(tokens)] = torch.tensor(tokens, dtype=torch.long)
        mask[row, :len(tokens)] = 1
    generated = [[] for _ in prompts]
    finished = [False] * len(prompts)
    hidden, cache = model.model(ids.to(dev), use_cache=True, attention_mask=mask.to(dev))
    last = hidden[torch.arange(len(prompts), device=dev), (lengths - 1).to(dev)]
    logits = model.lm_head(last)
    for step in range(max_new_tokens):
        tokens = logits.argmax(-1)
        for row, token in enumerate(tokens.tolist()):
            if finished[row]:
                continue
            generated[row].append(int(token))
            finished[row] = token == eos_token_id or bool(on_token and on_token(generated[row]))
        if all(finished) or step + 1 == max_new_tokens:
            break
        result = model(tokens[:, None], cache=cache, use_cache=True)
        cache = result["cache"]
        logits = result["logits"][:, -1]
    return generated
