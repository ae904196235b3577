"""LLMEngine: one `step()` is one scheduled forward pass.

The engine's interface is the reference's (vllmlite/engine.py:23-269):
`add_request`, `step() -> [RequestOutput]`, `has_work`, `abort`, `release`,
`get_text`, `generate`, `stats`, with a `runner` that implements the
`ModelRunner` boundary (vllmlite/runner.py:19-32). `EngineConfig.backend ==
"hip"` builds a `HipRunner`; any runner can be passed in instead.

A step, in the order whose observable effects (streams, step counts, stop
reasons) the reference fixes:
  1. the batcher schedules; requests it retired report as finished;
  2. the runner executes; when every row the step reads is consumed by a
     plain argmax (draft verification, or greedy sampling without a
     repetition penalty or a min_tokens EOS mask) and the runner can take
     the argmax itself (`execute_argmax`), it returns token ids instead of
     logits;
  3. per scheduled request: drafts are verified and dropped, the K/V written
     for the kept tokens is committed (publishing blocks that filled), and a
     request whose tokens all have K/V gets its new tokens, each checked
     against the stop rules (EOS / stop ids unless ignore_eos, max_tokens,
     stop strings on the text decoded up to the previous step, max_seq_len);
  4. with speculation on, running requests that are plain-decoding get up to
     k n-gram drafts within the token budget.

Lookahead (on by default, for runners that offer `launch_argmax` /
`collect`): while a greedy step runs on the device, the host already does
the next one's bookkeeping. After launching step n the engine applies the
part of step n's outcome that does not depend on the chosen tokens (K/V
commits, num_computed, one placeholder token per request that completes,
max_tokens / max_seq_len stops, which free blocks), schedules and launches
step n + 1 - a placeholder input token is the negative index of the row whose
argmax the device holds - and only then waits for step n's ids, writes them
over the placeholders, decodes text and reports. `step()` therefore returns
the outputs of the step launched by the call before. Lookahead is used only
for steps whose outcome cannot depend on token values: every row consumed by
a plain argmax, no stop strings, EOS and stop ids ignored (`ignore_eos`), no
speculation; any other step runs synchronously. Streams, step counts and
stop reasons are those of synchronous stepping.

`fork_request` starts a running copy of a request that shares all of its
blocks (the reference defines BlockManager.fork but no engine path calls it;
the copy-on-write workload uses it). Forking happens between synchronous
steps: drive it with `lookahead = False`.
"""

from __future__ import annotations

import itertools
import time
from typing import Dict, List, Optional

import numpy as np

from .batcher import Batcher, StepBatch
from .config import EngineConfig
from .request import Request, RequestOutput, SamplingParams, Status, finish_reason
from .runner import ModelRunner, make_runner
from .sampling import choose
from .speculative import NgramProposer, SpecStats, accept_greedy, verify
from .tokenizer import get_tokenizer


class LLMEngine:
    def __init__(self, cfg: Optional[EngineConfig] = None, tokenizer: Optional[str] = None,
                 speculative_tokens: int = 0, runner: Optional[ModelRunner] = None,
                 lookahead: bool = True):
        self.cfg = cfg or EngineConfig()
        self.tokenizer = get_tokenizer(tokenizer)
        self.spec_k = speculative_tokens
        self.proposer = NgramProposer(speculative_tokens) if speculative_tokens else None
        self.spec = SpecStats()
        if self.cfg.model.vocab_size < self.tokenizer.vocab_size:
            self.cfg.model.vocab_size = self.tokenizer.vocab_size
        self.runner = runner if runner is not None else make_runner(self.cfg)
        self.device_argmax = hasattr(self.runner, "execute_argmax")
        self.lookahead = lookahead
        self._inflight = None  # (batch, handle, emitted) of a launched, uncollected step
        self._next: Optional[StepBatch] = None  # scheduled, to run synchronously
        self.batcher = Batcher(self.cfg.scheduler, self.cfg.cache)
        self.seqs: Dict[str, Request] = {}
        self._ids = itertools.count()
        self.total_prompt_tokens = 0
        self.total_output_tokens = 0
        self.total_steps = 0
        self.busy_time = 0.0

    # ------------------------------------------------------------- requests --
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
        req = Request(rid, [int(t) for t in prompt_token_ids], params)
        self.seqs[rid] = req
        self.batcher.add(req)
        self.total_prompt_tokens += req.n_prompt
        return rid

    def abort(self, request_id: str) -> bool:
        return self.batcher.abort(request_id)

    def release(self, request_id: str) -> None:
        self.seqs.pop(request_id, None)

    def fork_request(self, parent_id: str, child_id: str) -> str:
        """A running copy of a running request, sharing all of its blocks,
        partial tail included; whichever of the two writes that tail first gets
        a copy-on-write pair."""
        if self._inflight is not None or self._next is not None:
            raise RuntimeError("fork_request needs synchronous steps: a lookahead step is in "
                               "flight (construct the engine with lookahead=False)")
        parent = self.seqs[parent_id]
        if parent not in self.batcher.running:
            raise ValueError(f"{parent_id} is not running")
        if child_id in self.seqs:
            raise ValueError(f"{child_id} exists")
        child = Request(child_id, parent.context_ids(), parent.params)
        child.n_prompt = parent.n_prompt
        child.num_computed = parent.num_computed
        child.status = parent.status
        child.first_token_at = parent.first_token_at
        child.text = parent.text
        self.batcher.fork(parent, child)
        self.batcher.running.append(child)
        self.seqs[child_id] = child
        return child_id

    def just_started(self, child_suffix: str):
        """(request id, K/V tokens written) of every running request, in running
        order, that has emitted exactly one token and is not itself a fork
        (id ending in child_suffix)."""
        return [(r.request_id, r.table.num_filled) for r in self.batcher.running
                if r.num_output == 1 and not r.request_id.endswith(child_suffix)]

    @property
    def has_work(self) -> bool:
        return self._inflight is not None or self._next is not None or self.batcher.has_work

    # ----------------------------------------------------------------- step --
    def _argmax_only(self, batch: StepBatch) -> bool:
        eos = self.tokenizer.eos_id
        for item in batch.scheduled:
            req = item.seq
            if req.n_draft:
                continue
            p = req.params
            if p.temperature != 0.0 or p.repetition_penalty != 1.0:
                return False
            if eos is not None and req.num_output < p.min_tokens:
                return False
        return True

    def _lookahead_ok(self, batch: StepBatch) -> bool:
        if not (self.lookahead and self.device_argmax and self.proposer is None
                and hasattr(self.runner, "launch_argmax")):
            return False
        eos = self.tokenizer.eos_id
        for item in batch.scheduled:
            p = item.seq.params
            if (p.temperature != 0.0 or p.repetition_penalty != 1.0 or p.stop
                    or item.seq.n_draft):
                return False
            if eos is not None and (not p.ignore_eos or item.seq.num_output < p.min_tokens):
                return False
        return True

    def _schedule(self) -> StepBatch:
        if self._next is not None:
            batch, self._next = self._next, None
            return self._drop_retired(batch)
        return self.batcher.schedule()

    @staticmethod
    def _drop_retired(batch: StepBatch) -> StepBatch:
        """A batch held since the previous call loses the requests retired in
        between (abort): their blocks went back to the pool, and so do the
        copy-on-write pairs whose destination was one of them."""
        if all(not item.seq.status.finished for item in batch.scheduled):
            return batch
        batch.scheduled = [i for i in batch.scheduled if not i.seq.status.finished]
        owned = {b for i in batch.scheduled for b in i.seq.table.block_ids}
        batch.cow = [(s, d) for s, d in batch.cow if d in owned]
        return batch

    def step(self) -> List[RequestOutput]:
        b = self.batcher
        if self._inflight is None:
            batch = self._schedule()
            outs = [self._finished_output(r) for r in b.drain_reports()]
            if not batch.scheduled:
                return outs
            if not self._lookahead_ok(batch):
                return outs + self._run_sync(batch)
            self._inflight = self._advance(self._launch(batch))
        else:
            outs = []
        # step n is on the device and advanced on the host: schedule n + 1
        nxt = self.batcher.schedule()
        # requests retired since step n was launched (aborted between calls,
        # or out of cache in this schedule) may hold one of its placeholders:
        # they are reported once the ids are in place, after step n's outputs
        retired = b.drain_reports()
        following = None
        if nxt.scheduled and self._lookahead_ok(nxt):
            following = self._launch(nxt)
        elif nxt.scheduled:
            self._next = nxt
        # step n's tokens replace its placeholders before step n + 1's outcome
        # is applied (publishing a block reads the tokens in it)
        outs += self._finish_launched(self._inflight)
        outs += [self._finished_output(r) for r in retired]
        self._inflight = self._advance(following) if following is not None else None
        return outs

    def _launch(self, batch: StepBatch):
        t0 = time.perf_counter()
        handle = self.runner.launch_argmax(batch)
        self.busy_time += time.perf_counter() - t0
        self.total_steps += 1
        return batch, handle

    def _advance(self, launched):
        """A launched greedy step's token-independent outcome."""
        batch, handle = launched
        rows = handle[0]
        b = self.batcher
        emitted = []
        for item, (row0, count) in zip(batch.scheduled, rows):
            req = item.seq
            b.commit(req, item.num_tokens)
            req.num_computed += item.num_tokens
            if req.num_computed < len(req.ids):
                continue  # a prefill chunk or a recompute, not finished yet
            req.append_token(-1 - (row0 + count - 1))  # the device holds its value
            self.total_output_tokens += 1
            p = req.params
            if req.num_output >= p.max_tokens:
                req.finish(Status.FINISHED_LENGTH, "length")
            elif len(req.ids) >= self.cfg.model.max_seq_len:
                req.finish(Status.FINISHED_LENGTH, "length")
            if req.status.finished:
                b.finish(req)
            # the output reports the request as this step left it: a later
            # retirement (abort, cache_full) is reported on its own afterwards
            emitted.append((req, len(req.ids) - 1, row0 + count - 1,
                            req.status.finished, req.stop_reason))
        return batch, handle, emitted

    def _finish_launched(self, inflight) -> List[RequestOutput]:
        """Wait for a launched step's ids; put them in place of the
        placeholders; report."""
        _, handle, emitted = inflight
        t0 = time.perf_counter()
        picks, _ = self.runner.collect(handle)
        self.busy_time += time.perf_counter() - t0
        outs = []
        for req, pos, row, finished, reason in emitted:
            tok = int(picks[row])
            req.ids[pos] = tok
            # a request preempted since holds its tokens; others also wait for
            # the next step's placeholder
            out = self._output(req, [tok], self._detok(req, [tok]))
            out.finished, out.finish_reason = finished, reason if finished else None
            outs.append(out)
        return outs

    def _run_sync(self, batch: StepBatch) -> List[RequestOutput]:
        b = self.batcher
        t0 = time.perf_counter()
        if self.device_argmax and self._argmax_only(batch):
            picks, rows = self.runner.execute_argmax(batch)
            logits = None
        else:
            logits, rows = self.runner.execute(batch)
            picks = None
        self.busy_time += time.perf_counter() - t0
        self.total_steps += 1
        eos = self.tokenizer.eos_id
        outs = []
        for item, (row0, count) in zip(batch.scheduled, rows):
            req = item.seq
            new = None
            if req.n_draft:
                drafts = req.draft_token_ids
                if picks is not None:
                    new, acc = accept_greedy(picks[row0:row0 + count], drafts)
                else:
                    new, acc = verify(logits[row0:row0 + count], drafts)
                req.clear_drafts()
                self.spec.proposed += len(drafts)
                self.spec.accepted += acc
                keep = acc + 1  # the rejected drafts' K/V is overwritten later
            else:
                keep = item.num_tokens
            b.commit(req, keep)
            req.num_computed += keep
            if req.num_computed < len(req.ids):
                continue  # a prefill chunk or a recompute, not finished yet
            if new is None:
                if picks is not None:
                    new = (int(picks[row0 + count - 1]),)
                else:
                    new = (self._sample(req, logits[row0 + count - 1], eos),)
            emitted = []
            for tok in new:
                req.append_token(tok)
                self.total_output_tokens += 1
                emitted.append(tok)
                self._stop_check(req, tok, eos)
                if req.status.finished:
                    break
            delta = self._detok(req, emitted)
            if req.status.finished:
                b.finish(req)
            outs.append(self._output(req, emitted, delta))
        if self.proposer is not None:
            self.spec.rounds += 1
            self._propose()
        return outs

    def _output(self, req: Request, emitted: List[int], delta: str) -> RequestOutput:
        return RequestOutput(
            request_id=req.request_id, token_ids=req.output_token_ids, new_token_ids=emitted,
            text_delta=delta, finished=req.status.finished,
            finish_reason=finish_reason(req.status), num_prompt_tokens=req.n_prompt,
            num_output_tokens=req.num_output, cached_prefix_tokens=req.cached_prefix_tokens)

    def _sample(self, req: Request, row: np.ndarray, eos) -> int:
        p = req.params
        if req.rng is None:
            req.rng = np.random.default_rng(p.seed)
        seen = req.context_ids() if p.repetition_penalty != 1.0 else ()
        return choose(row, p, seen, req.rng, req.num_output, eos)

    def _detok(self, req: Request, new: List[int]) -> str:
        if req.decoder is None:
            req.decoder = self.tokenizer.stream_decoder()
        delta = req.decoder(new)
        req.text += delta
        return delta

    def _stop_check(self, req: Request, tok: int, eos) -> None:
        p = req.params
        if not p.ignore_eos and (tok == eos or tok in p.stop_token_ids):
            req.finish(Status.FINISHED_STOP, "stop")
        elif req.num_output >= p.max_tokens:
            req.finish(Status.FINISHED_LENGTH, "length")
        elif p.stop and self._hit_stop_string(req, p.stop):
            req.finish(Status.FINISHED_STOP, "stop")
        elif len(req.ids) >= self.cfg.model.max_seq_len:
            req.finish(Status.FINISHED_LENGTH, "length")

    @staticmethod
    def _hit_stop_string(req: Request, stops) -> bool:
        """A stop string in the text decoded so far (up to the previous step's
        tokens) cuts the text there."""
        for s in stops:
            if s:
                at = req.text.find(s)
                if at >= 0:
                    req.text = req.text[:at]
                    return True
        return False

    def _propose(self) -> None:
        """Drafts for running requests that are plain-decoding, within the
        token budget left after one token per running request."""
        left = self.cfg.scheduler.max_batched_tokens - len(self.batcher.running)
        for req in self.batcher.running:
            if req.num_uncomputed != 1 or req.status.finished:
                continue
            room = min(self.spec_k, max(0, left))
            if room <= 0:
                break
            guess = self.proposer.propose(req, room)
            if guess:
                req.set_drafts(guess)
                left -= len(guess)
                self.spec.rounds_with_proposal += 1

    def _finished_output(self, req: Request) -> RequestOutput:
        return RequestOutput(
            request_id=req.request_id, token_ids=req.output_token_ids, new_token_ids=[],
            text_delta="", finished=True,
            finish_reason=req.stop_reason or finish_reason(req.status),
            num_prompt_tokens=req.n_prompt, num_output_tokens=req.num_output,
            cached_prefix_tokens=req.cached_prefix_tokens)

    # ------------------------------------------------------------- results --
    def get_text(self, request_id: str) -> str:
        return self.seqs[request_id].text

    def generate(self, prompts: List[str], params: Optional[SamplingParams] = None) -> List[str]:
        ids = [self.add_request(p, params) for p in prompts]
        while self.has_work:
            self.step()
        return [self.seqs[i].text for i in ids]

    def stats(self) -> dict:
        d = self.batcher.stats()
        d.update(steps=self.total_steps, prompt_tokens=self.total_prompt_tokens,
                 output_tokens=self.total_output_tokens, busy_seconds=round(self.busy_time, 4),
                 output_tokens_per_second=(self.total_output_tokens / self.busy_time
                                           if self.busy_time else 0.0))
        if self.proposer is not None:
            d.update(self.spec.as_dict())
        return d
