"""LLMEngine: one `step()` is one scheduled forward pass.

Behaviour follows vllmlite/engine.py:23-269: schedule, run the model runner,
verify drafts or sample, commit K/V, append tokens, check stops, detokenize,
then propose drafts for the next step. The only interface change is the
optional `runner` argument: the reference hard-codes its NumPy runner
(engine.py:46); here `EngineConfig.backend == "hip"` builds a `HipRunner`, and
any object implementing `ModelRunner` can be passed in instead.
"""

from __future__ import annotations

import itertools
import time
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from .config import EngineConfig
from .runner import ModelRunner, make_runner
from .sampling import sample
from .scheduler import Scheduler
from .sequence import RequestOutput, SamplingParams, Sequence, Status
from .speculative import NgramProposer, SpecStats, accept_greedy, verify
from .tokenizer import get_tokenizer


@dataclass
class _Detok:
    text: str = ""
    consumed: int = 0


class LLMEngine:
    def __init__(self, cfg: Optional[EngineConfig] = None, tokenizer: Optional[str] = None,
                 speculative_tokens: int = 0, runner: Optional[ModelRunner] = None):
        self.cfg = cfg or EngineConfig()
        self.tokenizer = get_tokenizer(tokenizer)
        self.spec_k = speculative_tokens
        self.proposer = NgramProposer(speculative_tokens) if speculative_tokens else None
        self.spec = SpecStats()
        if self.cfg.model.vocab_size < self.tokenizer.vocab_size:
            self.cfg.model.vocab_size = self.tokenizer.vocab_size
        self.runner = runner if runner is not None else make_runner(self.cfg)
        # greedy steps take the argmax on the runner's side when it offers one
        self.device_argmax = hasattr(self.runner, "execute_argmax")
        self.scheduler = Scheduler(self.cfg.scheduler, self.cfg.cache)
        self.seqs: Dict[str, Sequence] = {}
        self.detok: Dict[str, _Detok] = {}
        self.rngs: Dict[str, np.random.Generator] = {}
        self._ids = itertools.count()
        self.total_prompt_tokens = 0
        self.total_output_tokens = 0
        self.total_steps = 0
        self.busy_time = 0.0

    def next_request_id(self) -> str:
        return f"req-{next(self._ids)}"

    def add_request(self, prompt: Optional[str] = None, params: Optional[SamplingParams] = None,
                    request_id: Optional[str] = None,
                    prompt_token_ids: Optional[List[int]] = None) -> str:
        rid = request_id or self.next_request_id()
        params = params or SamplingParams()
        if prompt_token_ids is None:
            if prompt is None:
                raise ValueError("need prompt or prompt_token_ids")
            prompt_token_ids = self.tokenizer.encode(prompt)
        if not prompt_token_ids:
            raise ValueError("empty prompt")
        seq = Sequence(rid, [int(t) for t in prompt_token_ids], params)
        self.seqs[rid] = seq
        self.detok[rid] = _Detok()
        self.rngs[rid] = np.random.default_rng(params.seed)
        self.scheduler.add(seq)
        self.total_prompt_tokens += len(prompt_token_ids)
        return rid

    def abort(self, request_id: str) -> bool:
        return self.scheduler.abort(request_id)

    def fork_request(self, parent_id: str, child_id: str) -> str:
        """Start a running copy of a running request that shares all of its
        blocks, partial tail included (BlockManager.fork,
        vllmlite/block_manager.py:133-137; the reference defines the fork but
        no engine path calls it). The child's first write into the shared tail
        makes append_slots emit a copy-on-write pair. Used by the
        shared-prefix workload to exercise the CoW path."""
        parent = self.seqs[parent_id]
        if parent not in self.scheduler.running:
            raise ValueError(f"{parent_id} is not running")
        if child_id in self.seqs:
            raise ValueError(f"{child_id} exists")
        child = Sequence(child_id, list(parent.prompt_token_ids), parent.params)
        child.output_token_ids = list(parent.output_token_ids)
        child.num_computed = parent.num_computed
        child.status = parent.status
        child.first_token_at = parent.first_token_at
        self.scheduler.blocks.fork(parent, child)
        self.scheduler.blocks.live_tokens += child.table.num_filled
        self.scheduler.running.append(child)
        self.seqs[child_id] = child
        src = self.detok[parent_id]
        self.detok[child_id] = _Detok(src.text, src.consumed)
        self.rngs[child_id] = np.random.default_rng(parent.params.seed)
        return child_id

    def just_started(self, child_suffix: str):
        """(request id, KV tokens written) of every running request, in running
        order, that has emitted exactly one token and is not itself a fork
        (id ending in child_suffix)."""
        return [(s.request_id, s.table.num_filled) for s in self.scheduler.running
                if len(s.output_token_ids) == 1 and not s.request_id.endswith(child_suffix)]

    def release(self, request_id: str) -> None:
        self.seqs.pop(request_id, None)
        self.detok.pop(request_id, None)
        self.rngs.pop(request_id, None)

    @property
    def has_work(self) -> bool:
        return self.scheduler.has_work

    def _argmax_only(self, sched) -> bool:
        """True when every row the step's sequences read is used by a plain
        argmax: draft verification, or greedy sampling with no repetition
        penalty and no min_tokens EOS mask (sampling.sample's first branch)."""
        eos = self.tokenizer.eos_id
        for item in sched.scheduled:
            seq = item.seq
            if seq.draft_token_ids:
                continue
            p = seq.params
            if p.temperature != 0.0 or p.repetition_penalty != 1.0:
                return False
            if eos is not None and len(seq.output_token_ids) < p.min_tokens:
                return False
        return True

    def step(self) -> List[RequestOutput]:
        sched = self.scheduler.schedule()
        dropped = [self._retired_output(s) for s in self.scheduler.drain_reports()]
        if sched.is_empty:
            return dropped

        t0 = time.perf_counter()
        # a runner that can take the argmax on its side does so when every
        # row of the step is consumed by a plain argmax
        picked = None
        if self.device_argmax and self._argmax_only(sched):
            picked, rows = self.runner.execute_argmax(sched)
            logits = None
        else:
            logits, rows = self.runner.execute(sched)
        self.busy_time += time.perf_counter() - t0
        self.total_steps += 1

        results: List[RequestOutput] = dropped
        eos = self.tokenizer.eos_id
        blocks = self.scheduler.blocks
        for i, item in enumerate(sched.scheduled):
            seq = item.seq
            row0, count = rows[i]
            drafts = seq.draft_token_ids
            if drafts:
                drafts = list(drafts)
                if picked is not None:
                    new_tokens, accepted = accept_greedy(picked[row0:row0 + count], drafts)
                else:
                    new_tokens, accepted = verify(logits[row0:row0 + count], drafts)
                seq.draft_token_ids.clear()
                self.spec.proposed += len(drafts)
                self.spec.accepted += accepted
                # rejected drafts' K/V stays behind as garbage and is overwritten
                keep = accepted + 1
            else:
                new_tokens, keep = None, item.num_tokens

            blocks.commit(seq, keep)
            seq.num_computed += keep
            # chunked prefill / recompute land here before the prompt is done
            if seq.num_computed < seq.num_tokens:
                continue

            if new_tokens is None and picked is not None:
                new_tokens = [int(picked[row0 + count - 1])]
            elif new_tokens is None:
                # the seen-token list only matters under a repetition penalty
                seen = seq.token_ids if seq.params.repetition_penalty != 1.0 else ()
                new_tokens = [sample(logits[row0 + count - 1], seq.params, seen,
                                     self.rngs[seq.request_id], len(seq.output_token_ids), eos)]

            emitted = []
            for tok in new_tokens:
                seq.append_token(tok)
                self.total_output_tokens += 1
                emitted.append(tok)
                self._check_stop(seq, tok, eos)
                if seq.status.finished:
                    break

            delta = self._advance_detok(seq)
            if seq.status.finished:
                self.scheduler.finish(seq)
            results.append(RequestOutput(
                request_id=seq.request_id,
                token_ids=list(seq.output_token_ids),
                new_token_ids=emitted,
                text_delta=delta,
                finished=seq.status.finished,
                finish_reason=self._reason(seq),
                num_prompt_tokens=seq.num_prompt_tokens,
                num_output_tokens=len(seq.output_token_ids),
                cached_prefix_tokens=seq.cached_prefix_tokens,
            ))

        if self.proposer is not None:
            self.spec.rounds += 1
            self._make_proposals()
        return results

    def _make_proposals(self) -> None:
        """Draft tokens for sequences that are plain-decoding (engine.py:183-197)."""
        budget = self.cfg.scheduler.max_batched_tokens
        cost = len(self.scheduler.running)
        for seq in self.scheduler.running:
            if seq.num_uncomputed != 1 or seq.status.finished:
                continue
            room = min(self.spec_k, max(0, budget - cost))
            if room <= 0:
                break
            guess = self.proposer.propose(seq, room)
            if guess:
                seq.draft_token_ids = list(guess)
                cost += len(guess)
                self.spec.rounds_with_proposal += 1

    def _retired_output(self, seq: Sequence) -> RequestOutput:
        return RequestOutput(
            request_id=seq.request_id,
            token_ids=list(seq.output_token_ids),
            new_token_ids=[],
            text_delta="",
            finished=True,
            finish_reason=seq.stop_reason or self._reason(seq),
            num_prompt_tokens=seq.num_prompt_tokens,
            num_output_tokens=len(seq.output_token_ids),
            cached_prefix_tokens=seq.cached_prefix_tokens,
        )

    def _advance_detok(self, seq: Sequence) -> str:
        st = self.detok[seq.request_id]
        delta, st.consumed = self.tokenizer.decode_stream(seq.output_token_ids, st.consumed)
        st.text += delta
        return delta

    def _check_stop(self, seq: Sequence, tok: int, eos) -> None:
        p = seq.params
        if not p.ignore_eos and (tok == eos or tok in p.stop_token_ids):
            seq.finish(Status.FINISHED_STOP, "stop")
            return
        if len(seq.output_token_ids) >= p.max_tokens:
            seq.finish(Status.FINISHED_LENGTH, "length")
            return
        if p.stop:
            text = self.detok[seq.request_id].text
            for s in p.stop:
                if s and s in text:
                    self.detok[seq.request_id].text = text[:text.index(s)]
                    seq.finish(Status.FINISHED_STOP, "stop")
                    return
        if seq.num_tokens >= self.cfg.model.max_seq_len:
            seq.finish(Status.FINISHED_LENGTH, "length")

    @staticmethod
    def _reason(seq: Sequence) -> Optional[str]:
        return {Status.FINISHED_STOP: "stop", Status.FINISHED_LENGTH: "length",
                Status.ABORTED: "abort"}.get(seq.status)

    def get_text(self, request_id: str) -> str:
        return self.detok[request_id].text

    def generate(self, prompts: List[str], params: Optional[SamplingParams] = None) -> List[str]:
        ids = [self.add_request(p, params) for p in prompts]
        while self.has_work:
            self.step()
        return [self.detok[i].text for i in ids]

    def stats(self) -> dict:
        d = self.scheduler.stats()
        d.update(
            steps=self.total_steps,
            prompt_tokens=self.total_prompt_tokens,
            output_tokens=self.total_output_tokens,
            busy_seconds=round(self.busy_time, 4),
            output_tokens_per_second=(self.total_output_tokens / self.busy_time
                                      if self.busy_time else 0.0),
        )
        if self.proposer is not None:
            d.update(self.spec.as_dict())
        return d
