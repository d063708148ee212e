"""Token-level generation loop, mirroring crates/esp/src/infer/decoder/generate.rs.

Prefill the prompt once, then KV-cached single-token steps; each token is
chosen by a `TokenPicker` (greedy argmax, lowest id on ties, or a seeded
`Sampler`). Both pickers run on the device (`esp_pick`). A greedy run with
no per-token callback executes as one device-resident loop
(`esp_generate_greedy`): same tokens, no host round trip per step.
"""
from __future__ import annotations

from typing import Callable, List, Optional, Sequence, Tuple

from .model import DecoderModel, KvCache
from .sample import Sampler


class TokenPicker:
    """generate.rs:21-64. `TokenPicker.greedy()` or `TokenPicker.sampled(sampler)`."""

    def __init__(self, sampler: Optional[Sampler] = None):
        self.sampler = sampler

    @staticmethod
    def greedy() -> "TokenPicker":
        return TokenPicker(None)

    @staticmethod
    def sampled(sampler: Sampler) -> "TokenPicker":
        return TokenPicker(sampler)

    def pick(self, model: DecoderModel, cache: KvCache) -> int:
        """generate.rs:30-44 over the last forward's device-resident logits."""
        ids, _ = model.pick(cache, 1, None, None if self.sampler is None else [self.sampler])
        return int(ids[0])


def generate_ids(model: DecoderModel, prompt_ids: Sequence[int], max_new: int,
                 eos: Sequence[int], on_token: Optional[Callable[[int], bool]] = None) -> List[int]:
    """generate.rs:98-114 (greedy)."""
    return generate_ids_with(model, prompt_ids, max_new, eos, TokenPicker.greedy(), on_token)


def generate_ids_with(model: DecoderModel, prompt_ids: Sequence[int], max_new: int,
                      eos: Sequence[int], picker: TokenPicker,
                      on_token: Optional[Callable[[int], bool]] = None) -> List[int]:
    """generate.rs:116-129 -> try_generate_ids_with."""
    return try_generate_ids_with(model, prompt_ids, max_new, eos, picker, on_token)


def try_generate_ids_with(model: DecoderModel, prompt_ids: Sequence[int], max_new: int,
                          eos: Sequence[int], picker: TokenPicker,
                          on_token: Optional[Callable[[int], bool]] = None,
                          cache: Optional[KvCache] = None) -> List[int]:
    """generate.rs:134-170. `on_token(id)` returning True stops after that id
    (the reference's ControlFlow::Break). Returns the generated ids, prompt
    and eos excluded."""
    if not prompt_ids:
        raise AssertionError("prompt must not be empty")
    # The reference's cache grows; a forward past the window is refused when
    # it is taken (model.rs:547-556), so a run that ends at eos first
    # succeeds. The cache is sized to the window at most.
    need = len(prompt_ids) + max(0, max_new - 1)
    cache = cache or model.new_cache(1, max(1, min(need, model.config.max_position_embeddings)))
    if picker.sampler is None and on_token is None:
        return model.generate_greedy_device(cache, prompt_ids, max_new, eos)
    cache.reset(0)
    model.try_forward_cached_last(prompt_ids, cache)
    out: List[int] = []
    for position in range(max_new):
        token = picker.pick(model, cache)
        if token in eos:
            break
        out.append(token)
        stop = bool(on_token(token)) if on_token is not None else False
        if stop or position + 1 == max_new:
            break
        model.try_forward_cached_last([token], cache)
    return out


def generate_constrained(model: DecoderModel, prompt_ids: Sequence[int], max_new: int,
                         eos: Sequence[int], picker: TokenPicker, constraint, tokenizer,
                         cache: Optional[KvCache] = None) -> Tuple[List[int], bool]:
    """The token loop of provider.rs:735-883 under an output grammar.

    Each turn either takes the grammar's forced span (constraint.rs:296-344;
    a sampled picker skips one draw per forced token, provider.rs:819-824)
    or picks one token from the logits masked on the device by the
    constraint (provider.rs:744-817), with the reference's recovery from
    non-finite scores (one recompute of the prefix, then Backend;
    provider.rs:219-240). Tokens are accepted into the constraint; the loop
    ends when the grammar is complete or an eos id is picked, and a token
    limit reached first is InvalidRequest (provider.rs:874-878). Forced
    spans are evaluated as one block over the warm cache. Returns
    (ids, complete)."""
    from .provider import DecoderProvider, GenerationCheckpoint
    if not prompt_ids:
        raise AssertionError("prompt must not be empty")
    need = len(prompt_ids) + max(0, max_new - 1)
    cache = cache or model.new_cache(1, max(1, min(need, model.config.max_position_embeddings)))
    cache.reset(0)
    model.try_forward_cached_last(list(prompt_ids), cache)
    provider = DecoderProvider(model, eos, tokenizer)
    cp = GenerationCheckpoint(request=None, prompt_ids=list(prompt_ids), token_ids=[], draws=0,
                              complete=False)
    provider._token_loop(cache, cp, max_new, picker, constraint, lambda _: None, lambda: False)
    return list(cp.token_ids), cp.complete
