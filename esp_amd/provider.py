"""Durable, id-level generation: the decoder provider's checkpointed loop.

Mirrors `DecoderProvider` of crates/esp/src/infer/decoder/provider.rs at the
token-id seam: request admission and the window rule (`prepare_generation`,
provider.rs:474-517), the resumable loop with commit and stop callbacks at
token boundaries (`generate_checkpointed`, provider.rs:612-883), and the
numerical-recovery rule for non-finite scores (`finite_score_row`,
provider.rs:219-240, used at :744-806).

Every forward, mask and token choice runs on the device through the C ABI;
this module keeps the host state the reference keeps: the committed ids,
the draw count, the grammar automaton and the sampler's RNG state. Text
(tokenisation of the prompt, streaming detokenisation, stop strings and the
checkpoint's `text` field) is host string work above this seam: requests
carry prompt ids, and a request with stop strings is refused as
Unsupported. A tokenizer is only needed for grammar-forced spans
(constraint.rs:296-344).
"""
from __future__ import annotations

import copy
import math
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence, Tuple

from .errors import Backend, InvalidRequest, PromptTooLong, Unsupported
from .generate import TokenPicker, try_generate_ids_with
from .model import DecoderModel, KvCache
from .sample import Sampler, SplitMix64

ESP_PICK_NONFINITE = 1  # include/esp_hip.h: the row held NaN / inf scores


@dataclass
class GenerationRequest:
    """provider.rs:91-117 `GenerationRequest` with the prompt as token ids."""

    prompt_ids: List[int]
    max_tokens: int
    temperature: float = 0.0
    top_p: Optional[float] = None
    seed: Optional[int] = None
    output_grammar: Optional[dict] = None
    stop: List[str] = field(default_factory=list)


@dataclass
class GenerationCheckpoint:
    """provider.rs:219-231 `GenerationCheckpoint` without the text, session
    and placement fields (host string and session state above this seam)."""

    request: GenerationRequest
    prompt_ids: List[int]
    token_ids: List[int]
    draws: int
    complete: bool


@dataclass
class ScoreHealth:
    """provider.rs:35-42: numerical observations of checkpointed calls."""

    checked_rows: int = 0
    invalid_rows: int = 0
    prefix_recomputations: int = 0
    failed_recoveries: int = 0


class DecoderProvider:
    """provider.rs:62-72 `DecoderProvider` over a loaded `DecoderModel`.

    `eos_token_ids` end generation (excluded from the output); the context
    window is the model's `max_position_embeddings` (provider.rs:271).
    `tokenizer` (a `tokenizers.Tokenizer`) and `vocab` (a shared
    `Vocabulary`) serve output grammars."""

    def __init__(self, model: DecoderModel, eos_token_ids: Sequence[int] = (),
                 tokenizer=None, vocab=None):
        self.model = model
        self.eos_token_ids = list(eos_token_ids)
        self.context_window = model.config.max_position_embeddings
        self.tokenizer = tokenizer
        self._vocab = vocab
        self._health = ScoreHealth()

    def score_health(self) -> ScoreHealth:
        """provider.rs:309-320"""
        return copy.copy(self._health)

    # -- request admission ------------------------------------------------

    def prepare_generation(self, request: GenerationRequest) -> Tuple[List[int], int, TokenPicker]:
        """provider.rs:474-517: refusals, the picker, and the window rule
        `max_new = min(max_tokens, window - prompt)`."""
        if not request.prompt_ids:
            raise InvalidRequest("empty prompt")
        if request.max_tokens == 0:
            raise InvalidRequest("max_tokens is 0")
        t = request.temperature
        if t < 0.0 or not math.isfinite(t):
            raise InvalidRequest(f"temperature must be finite and >= 0, got {t}")
        if t == 0.0:
            picker = TokenPicker.greedy()
        else:
            seed = request.seed if request.seed is not None else SplitMix64.from_entropy()[1]
            picker = TokenPicker.sampled(Sampler(t, request.top_p, seed))
        prompt_ids = [int(i) for i in request.prompt_ids]
        window = self.context_window
        if len(prompt_ids) >= window:
            raise PromptTooLong(len(prompt_ids), window)
        return prompt_ids, min(request.max_tokens, window - len(prompt_ids)), picker

    def _constraint(self, request: GenerationRequest):
        if request.output_grammar is None:
            return None
        if request.stop:
            raise InvalidRequest("stop strings cannot truncate constrained output")
        from .constraint import Constraint, Vocabulary
        if self._vocab is None:
            if self.tokenizer is None:
                raise InvalidRequest("constraint needs a tokenizer and vocabulary size")
            self._vocab = Vocabulary.from_tokenizer(self.tokenizer, self.model.config.vocab_size)
        return Constraint(request.output_grammar, vocab=self._vocab)

    # -- plain generation -------------------------------------------------

    def generate_ids(self, request: GenerationRequest,
                     on_token: Optional[Callable[[int], bool]] = None) -> List[int]:
        """provider.rs:519-557 `generate_streaming_observed` at the id seam:
        generated ids (prompt and eos excluded). `on_token(id)` returning
        True stops after that id."""
        if request.stop:
            raise Unsupported("stop", "stop strings need the detokenizer above this seam")
        if request.output_grammar is not None:
            stopped = [False]
            seen = [0]

            def commit(cp: GenerationCheckpoint) -> None:
                for t in cp.token_ids[seen[0]:]:
                    if on_token is not None and on_token(t):
                        stopped[0] = True
                seen[0] = len(cp.token_ids)

            return list(self.generate_checkpointed(request, None, commit,
                                                   lambda: stopped[0]).token_ids)
        prompt_ids, max_new, picker = self.prepare_generation(request)
        return try_generate_ids_with(self.model, prompt_ids, max_new, self.eos_token_ids,
                                     picker, on_token)

    # -- durable generation -----------------------------------------------

    def generate_checkpointed(self, request: GenerationRequest,
                              resume: Optional[GenerationCheckpoint] = None,
                              commit: Optional[Callable[[GenerationCheckpoint], None]] = None,
                              stop: Optional[Callable[[], bool]] = None) -> GenerationCheckpoint:
        """provider.rs:612-883. `commit(cp)` sees every token boundary (an
        exception from it ends the call before another token); `stop()`
        pauses at a boundary without spending a draw. Resuming from a paused
        checkpoint re-prefills prompt + committed ids, replays them into the
        grammar and skips the recorded draws, so the stream continues as if
        never paused."""
        commit = commit or (lambda cp: None)
        stop = stop or (lambda: False)
        if request.stop:
            raise Unsupported("stop", "stop strings need the detokenizer above this seam")
        if resume is not None:
            supplied = copy.deepcopy(request)
            if supplied.temperature > 0.0 and supplied.seed is None:
                supplied.seed = resume.request.seed
            if resume.request != supplied:
                raise InvalidRequest("checkpoint request differs from supplied request")
        request = copy.deepcopy(resume.request if resume is not None else request)
        if request.temperature > 0.0 and request.seed is None:
            request.seed = SplitMix64.from_entropy()[1]
        prompt_ids, max_new, picker = self.prepare_generation(request)
        if resume is not None:
            cp = copy.deepcopy(resume)
        else:
            cp = GenerationCheckpoint(request=copy.deepcopy(request), prompt_ids=list(prompt_ids),
                                      token_ids=[], draws=0, complete=False)
        sampled = request.temperature > 0.0
        vocab = self.model.config.vocab_size
        if (cp.prompt_ids != prompt_ids or len(cp.token_ids) > max_new
                or any(not 0 <= t < vocab for t in cp.token_ids)
                or (not cp.complete and cp.draws != (len(cp.token_ids) if sampled else 0))):
            raise InvalidRequest("invalid generation checkpoint tokens or draw position")
        constraint = self._constraint(request)
        if constraint is not None:
            for t in cp.token_ids:
                constraint.accept(t)
            if cp.complete and not constraint.complete():
                raise InvalidRequest("complete checkpoint violates output grammar")
        if cp.complete:
            return cp
        if picker.sampler is not None:
            picker.sampler.skip_draws(cp.draws)
        commit(cp)
        if stop():
            return cp
        prefix = prompt_ids + cp.token_ids
        if len(prefix) >= self.context_window:
            raise PromptTooLong(len(prefix), self.context_window)
        cache = self.model.new_cache(1, min(len(prefix) + max_new - len(cp.token_ids),
                                            self.context_window))
        self.model.try_forward_cached_last(prefix, cache)
        self._token_loop(cache, cp, max_new, picker, constraint, commit, stop)
        return cp

    def _token_loop(self, cache: KvCache, cp: GenerationCheckpoint, max_new: int,
                    picker: TokenPicker, constraint, commit: Callable[[GenerationCheckpoint], None],
                    stop: Callable[[], bool]) -> None:
        """provider.rs:735-880 over a cache holding prompt + committed ids:
        forced spans or one device pick per turn, each token committed at
        its boundary, ended by eos, grammar completion, the token limit or
        `stop()`. Updates `cp` in place."""
        sampler = picker.sampler
        sampled = sampler is not None
        recovery_used = [False]
        while len(cp.token_ids) < max_new:
            if stop():
                return
            forced = constraint.forced(self.tokenizer) if constraint is not None else []
            if forced:
                # forced syntax consumes the same recorded draw positions on
                # replay (provider.rs:819-824)
                if sampler is not None:
                    sampler.skip_draws(len(forced))
                tokens = forced
            elif constraint is not None:
                token = self._pick_finite(cache, constraint, sampler, cp, recovery_used, stop)
                if token is None:
                    return
                tokens = [token]
            else:
                tokens = [picker.pick(self.model, cache)]
            evaluated: List[int] = []
            for token in tokens[:max_new - len(cp.token_ids)]:
                if stop():
                    return
                cp.draws += int(sampled)
                if token in self.eos_token_ids:
                    cp.complete = True
                else:
                    if constraint is not None:
                        constraint.accept(token)
                    cp.token_ids.append(token)
                    evaluated.append(token)
                    cp.complete = (constraint.complete() if constraint is not None
                                   else len(cp.token_ids) == max_new)
                commit(cp)
                if cp.complete or stop():
                    return
            if len(cp.token_ids) == max_new:
                break
            self.model.try_forward_cached_last(evaluated, cache)
        if constraint is not None:
            raise InvalidRequest("token limit reached before output grammar completed")
        cp.complete = True
        commit(cp)

    def _observe_scores(self, cache: KvCache, index: int) -> None:
        """Called before each constrained token choice with the number of
        committed output ids; the scores are the device logits row of
        `cache`. A no-op here: the place where provider.rs's test build
        substitutes fault rows (provider.rs:70-71, 755-762)."""

    def _pick_finite(self, cache: KvCache, constraint, sampler: Optional[Sampler],
                     cp: GenerationCheckpoint, recovery_used: List[bool],
                     stop: Callable[[], bool]) -> Optional[int]:
        """provider.rs:744-817 with `finite_score_row` (provider.rs:219-240):
        a row holding NaN or inf never becomes a token decision. The first
        such row of a call rebuilds the committed prefix on a fresh cache
        once; a second one, or a recomputed row that is still non-finite,
        fails closed with Backend. The pick is made on the device, so a
        flagged pick is discarded and the sampler's state restored: no draw
        is spent on it. Returns None when `stop()` asks to pause."""
        self._observe_scores(cache, len(cp.token_ids))
        samplers = None if sampler is None else [sampler]
        state = None if sampler is None else sampler.rng.state
        ids, flags, status = self.model.pick_constrained(cache, [constraint], samplers,
                                                         check=False)
        if flags[0] & ESP_PICK_NONFINITE:
            if sampler is not None:
                sampler.rng.state = state
            if stop():
                return None
            self._health.checked_rows += 1
            self._health.invalid_rows += 1
            if recovery_used[0]:
                self._health.failed_recoveries += 1
                raise Backend("non-finite model scores after numerical recovery was already used")
            recovery_used[0] = True
            self._health.prefix_recomputations += 1
            cache.reset(0)
            self.model.try_forward_cached_last(cp.prompt_ids + cp.token_ids, cache)
            ids, flags, status = self.model.pick_constrained(cache, [constraint], samplers,
                                                             check=False)
            self._health.checked_rows += 1
            if flags[0] & ESP_PICK_NONFINITE:
                self._health.invalid_rows += 1
                self._health.failed_recoveries += 1
                if sampler is not None:
                    sampler.rng.state = state
                raise Backend("recomputed model scores are non-finite or have changed "
                              "vocabulary size")
        else:
            self._health.checked_rows += 1
        from . import _lib
        _lib.check(status)
        return int(ids[0])
