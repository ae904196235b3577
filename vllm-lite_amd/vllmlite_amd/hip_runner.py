"""HipRunner: the ModelRunner boundary (vllmlite/runner.py:19-100) on one MI355X.

execute(SchedulerOutput) -> (logits, rows), exactly as the reference's
NumpyRunner: logits is a host float32 array [R, vocab], rows[i] = (first_row,
count) for scheduled sequence i, count = min(1 + drafts, tokens)
(runner.py:86-90). Per call:

  1. copy-on-write pairs, in list order, before any K/V write
     (runner.py:54-64): one vl_copy_blocks launch over all layers;
  2. the ragged batch is flattened on the host into one int32 record
     [token_ids | positions | slot_mapping | logits_idx | query_start_loc |
     seq_lens | block_tables] (runner.py:62-100, block.py:154-156) and sent
     with a single host-to-device copy from pinned memory;
  3. the TinyLlama forward (model.py:80-120) runs on the device. Steps of up
     to FUSED_ROWS_MAX tokens (every step of the published mixes) run each
     projection as one vl_linear_rows / vl_qkv_rope_cache launch over 16-row
     tiles, with the RMSNorm before it and the residual add, SwiGLU, or RoPE
     and the K/V slot scatter after it fused in (weights in 16-column tiles;
     layer 0 also gathers the embedding rows), and the ragged paged attention
     between (planned once per step, run per layer; decode-only steps take
     the short-decode kernel, no plan); finally RMSNorm and the lm_head on the
     logits rows only. Larger steps run PyTorch GEMMs with separate RMSNorm,
     RoPE + scatter and SwiGLU launches;
  4. one device-to-host copy of the logits rows and a stream synchronisation
     (execute), or the argmax of each row written to pinned host memory by
     its launch (execute_argmax / launch_argmax).

With one_launch_decode = True, a decode step of at most 16 sequences
(every sequence one query token) whose model shape has a one-launch kernel
(ops.decode_step_supported) runs instead as ONE launch, vl_decode_step, on
the compute units of one XCD: the whole forward, the logits rows and the
argmax of each row, written to device memory and to the pinned host buffer of
the step. Its logits agree with the separate kernels' to ~1e-6 (the
attention sums in another order); it is off by default because on the
48-request mix it takes longer per step (268 against 202 us).

Step 3 is otherwise captured once per shape bucket (tokens, sequences and logits rows
each rounded up to a power of two) into a HIP graph and replayed afterwards;
padded tokens belong to no sequence, carry slot -1 (no cache write) and
position 0, padded sequences have no tokens and no context, and the rows they
produce are never read. The larger steps' GEMMs are PyTorch (hipBLASLt) in fp32
with TF32-style reduced precision off; everything else is the gfx950 library.

The engine calls execute serially, possibly from a different thread each time
(async_engine.py:47): every call selects the runner's device and stream.
"""

from __future__ import annotations

import gc
from typing import Dict, List, Tuple

import numpy as np
import torch

from . import ops
from .model import model_weights, pack_weights, rope_tables, tile_weights
from .runner import ModelRunner


# steps of at most this many token rows run the fused projection kernels
# (vl_linear_rows, vl_qkv_rope_cache: 16-row tiles, norm / residual / SwiGLU /
# RoPE + scatter inside); larger ones hipBLASLt GEMMs and separate launches
FUSED_ROWS_MAX = 1024


def _bucket(n: int, floor: int) -> int:
    b = floor
    while b < n:
        b *= 2
    return b


class Flattened:
    """One step's ragged batch as plain int lists, in schedule order."""

    __slots__ = ("toks", "pos", "slots", "lidx", "qsl", "lens", "tables", "rows", "T", "S",
                 "R", "width", "max_q")


def flatten_scheduled(out, block_size: int, max_seq_len: int) -> Flattened:
    """SchedulerOutput -> Flattened (vllmlite/runner.py:62-100), reading only
    the fields the reference runner reads: `item.start_pos` and
    `item.num_tokens` of each scheduled item (scheduler.py:23-30),
    `seq.token_ids[start:start + n]`, `seq.draft_token_ids` and
    `seq.table.block_ids` (sequence.py:49-94, block.py:120-156). A sequence
    object may offer `token_slice(start, stop)` to skip building the whole
    token list. Sequence i contributes positions start..start+n-1, slots
    block_ids[p // bs] * bs + p % bs (block.py:154-156) and the last
    min(1 + drafts, n) token rows as logits rows (runner.py:86-90)."""
    bs = block_size
    f = Flattened()
    toks: List[int] = []
    pos: List[int] = []
    slots: List[int] = []
    lidx: List[int] = []
    qsl: List[int] = [0]
    lens: List[int] = []
    rows: List[Tuple[int, int]] = []
    tables = []
    T = R = max_q = 0
    width = 1
    for item in out.scheduled:
        seq = item.seq
        st, n = item.start_pos, item.num_tokens
        ids = seq.table.block_ids
        nb = len(ids)
        end = st + n
        if end > nb * bs:
            raise ValueError(f"sequence {seq.request_id}: {end} tokens but only {nb} blocks")
        if end > max_seq_len:
            # the reference fails the same way indexing its RoPE table
            raise IndexError(f"position {end - 1} beyond max_seq_len {max_seq_len}")
        fast = getattr(seq, "token_slice", None)
        toks += fast(st, end) if fast is not None else seq.token_ids[st:end]
        if n == 1:
            pos.append(st)
            slots.append(ids[st // bs] * bs + st % bs)
        else:
            p = range(st, end)
            pos += p
            slots += [ids[q // bs] * bs + q % bs for q in p]
        c = min(1 + len(seq.draft_token_ids), n)
        lidx += range(T + n - c, T + n)
        rows.append((R, c))
        T += n
        R += c
        qsl.append(T)
        lens.append(end)
        tables.append(ids)
        if nb > width:
            width = nb
        if n > max_q:
            max_q = n
    f.toks, f.pos, f.slots, f.lidx, f.qsl, f.lens = toks, pos, slots, lidx, qsl, lens
    f.tables, f.rows, f.T, f.S, f.R, f.width = tables, rows, T, len(tables), R, width
    f.max_q = max_q
    return f


def fused_rows_supported(mc) -> bool:
    """Steps of up to FUSED_ROWS_MAX token rows run the fused projection
    kernels (vl_linear_rows, vl_qkv_rope_cache), which need d_model and d_ff to be
    multiples of 16 within their K limits; other shapes take the GEMM path for
    every step and keep no tiled weight copies."""
    return (mc.d_model % 16 == 0 and mc.d_ff % 16 == 0 and mc.d_model <= 512
            and mc.d_ff <= 1024)


class _Shape:
    """Offsets of one bucket's int32 record and views of the device buffers."""

    def __init__(self, Tb: int, Sb: int, Rb: int, W: int, decode: bool = False):
        # decode: every sequence has one query (its attention takes the
        # short-decode kernel, which needs no plan)
        self.Tb, self.Sb, self.Rb, self.W, self.decode = Tb, Sb, Rb, W, decode
        o = 0
        self.tok, o = o, o + Tb
        self.pos, o = o, o + Tb
        self.slot, o = o, o + Tb
        self.lidx, o = o, o + Rb
        self.qsl, o = o, o + Sb + 1
        self.lens, o = o, o + Sb
        self.bt, o = o, o + Sb * W
        self.n_ints = o


class RecordStager:
    """Writes a step's ragged batch into an int32 record (the layout of
    _Shape) that alternates between `nbuf` host buffers, with the same
    contents flatten_scheduled gives, in fewer host operations: the per-token
    and per-sequence segments as one list converted once, and the block
    tables incrementally. A block-table row is rewritten only when its
    sequence's table is another list than the one this buffer last held at
    that row (a different or re-admitted sequence), or the table shrank;
    when it grew, only the new entries are written. Entries past a row's
    table are never read (its length bounds every read), so they are left
    as they are. A step with copy-on-write pairs (block ids replaced inside a
    table) and any change of the record's layout rewrite every row. Converting
    the whole table region each step (Sb x W ints, 512 for the 48-request mix)
    cost 10-18 us of host time per step."""

    def __init__(self, nbuf: int = 2):
        self._rows = [[] for _ in range(nbuf)]  # per buffer: [table list, entries written]
        self._layout = [None] * nbuf            # per buffer: (bt offset, W) of its rows

    def reset(self) -> None:
        """The host buffers were replaced: nothing in them is known."""
        for k in range(len(self._rows)):
            self._rows[k] = []
            self._layout[k] = None

    def stage(self, out, m: np.ndarray, k: int, block_size: int, max_seq_len: int, W: int,
              short_decode: bool, cap_T: int):
        """Record of `out` into m (buffer k, sized for cap_T tokens and W
        blocks per table). Returns (shape, rows, R, T, width); shape is None,
        and nothing is written, when the step needs more room."""
        bs = block_size
        toks: List[int] = []
        pos: List[int] = []
        slots: List[int] = []
        lidx: List[int] = []
        qsl: List[int] = [0]
        lens: List[int] = []
        rows: List[Tuple[int, int]] = []
        tables = []
        T = R = max_q = 0
        width = 1
        for item in out.scheduled:
            seq = item.seq
            st, n = item.start_pos, item.num_tokens
            ids = seq.table.block_ids
            nb = len(ids)
            end = st + n
            if end > nb * bs:
                raise ValueError(f"sequence {seq.request_id}: {end} tokens but only {nb} blocks")
            if end > max_seq_len:
                raise IndexError(f"position {end - 1} beyond max_seq_len {max_seq_len}")
            fast = getattr(seq, "token_slice", None)
            toks += fast(st, end) if fast is not None else seq.token_ids[st:end]
            if n == 1:
                pos.append(st)
                slots.append(ids[st // bs] * bs + st % bs)
            else:
                pos += range(st, end)
                slots += [ids[q // bs] * bs + q % bs for q in range(st, end)]
            c = min(1 + len(seq.draft_token_ids), n)
            lidx += range(T + n - c, T + n)
            rows.append((R, c))
            T += n
            R += c
            qsl.append(T)
            lens.append(end)
            tables.append(ids)
            if nb > width:
                width = nb
            if n > max_q:
                max_q = n
        S = len(tables)
        if width > W or T > cap_T:
            return None, rows, R, T, width  # the caller grows the buffers and stages again
        shape = _Shape(_bucket(T, 16), _bucket(S, 8), _bucket(R, 8), W,
                       max_q == 1 and short_decode)
        Tb, Sb, Rb = shape.Tb, shape.Sb, shape.Rb
        head = (toks + [0] * (Tb - T) + pos + [0] * (Tb - T) + slots + [-1] * (Tb - T) +
                lidx + [0] * (Rb - R) + qsl + [T] * (Sb - S) + lens + [0] * (Sb - S))
        m[:shape.bt] = head
        known = self._rows[k]
        if getattr(out, "cow", None) or self._layout[k] != (shape.bt, W):
            self._layout[k] = (shape.bt, W)
            known = self._rows[k] = []
        while len(known) < S:
            known.append([None, 0])
        base = shape.bt
        for i, ids in enumerate(tables):
            kr = known[i]
            nb = len(ids)
            if kr[0] is ids and kr[1] <= nb:
                if kr[1] < nb:
                    m[base + i * W + kr[1]:base + i * W + nb] = ids[kr[1]:]
            else:
                m[base + i * W:base + i * W + nb] = ids
                kr[0] = ids
            kr[1] = nb
        return shape, rows, R, T, width


class HipRunner(ModelRunner):
    def __init__(self, model_cfg, cache_cfg, weights: Dict[str, np.ndarray] = None,
                 device=None, use_graphs: bool = True, one_launch_decode: bool = False,
                 fused_wo: bool = True):
        if not torch.cuda.is_available():
            raise RuntimeError("HipRunner needs a visible MI355X (torch.cuda.is_available() is False)")
        ops.lib()  # fail now, loudly, if the gfx950 library is not built
        torch.backends.cuda.matmul.allow_tf32 = False
        self.model_cfg = model_cfg
        self.cache_cfg = cache_cfg
        self.block_size = cache_cfg.block_size
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        self.use_graphs = use_graphs
        mc = model_cfg
        self.H, self.Hkv, self.hd = mc.n_heads, mc.n_kv_heads, mc.head_dim
        self.scale = float(1.0 / np.sqrt(mc.head_dim))
        with torch.cuda.device(self.device):
            self.stream = torch.cuda.Stream(self.device)
            w = weights if weights is not None else model_weights(mc)
            self.w = pack_weights(mc, w, torch, self.device)
            self._fused_rows = fused_rows_supported(mc)
            self.fused_rows_max = FUSED_ROWS_MAX
            if self._fused_rows:
                tile_weights(self.w, ops.tile16, torch)
            cos, sin = rope_tables(mc.head_dim, mc.max_seq_len)
            self.cos = torch.from_numpy(cos).to(self.device)
            self.sin = torch.from_numpy(sin).to(self.device)
            slots = cache_cfg.num_blocks * cache_cfg.block_size
            if getattr(cache_cfg, "kv_layout", "token") == "head":
                shape = (mc.n_layers, cache_cfg.num_blocks, mc.n_kv_heads, cache_cfg.block_size,
                         mc.head_dim)
            else:
                shape = (mc.n_layers, slots, mc.n_kv_heads, mc.head_dim)
            kv = {"bfloat16": torch.bfloat16, "float8_e4m3": torch.float8_e4m3fn}.get(
                getattr(cache_cfg, "kv_dtype", "float32"), torch.float32)
            self.cache_k = torch.zeros(shape, dtype=kv, device=self.device)
            self.cache_v = torch.zeros(shape, dtype=kv, device=self.device)
            # decode steps of <= 16 sequences as one launch, where a kernel exists
            self._step = None
            self.one_launch_steps = 0
            if (one_launch_decode and self._fused_rows and ops.decode_step_supported(
                    mc.d_model, mc.n_heads, mc.n_kv_heads, mc.d_ff, kv, mc.max_seq_len)):
                self._step = ops.DecodeStep(self.w, self.device)
                self._exec_ids_host = torch.zeros(ops.DECODE_STEP_ROWS + 1, dtype=torch.int32,
                                                  pin_memory=True)
        self.W = max(1, -(-mc.max_seq_len // self.block_size))
        self._buf = 0  # which of the two pinned staging / id buffers the next launch uses
        self._stager = RecordStager(2)
        self._cap_T = 0
        self._graphs: Dict[Tuple[int, int, int, bool, int], torch.cuda.CUDAGraph] = {}
        self._graph_exec: Dict[Tuple[int, int, int, bool, int], int] = {}  # raw exec handles
        self._dev_index = (self.device.index if self.device.index is not None
                           else torch.cuda.current_device())
        self._stream_h = self.stream.cuda_stream
        # captured steps are launched from the library's submission thread
        # (hipGraphLaunch costs the caller ~1 us per node); anything this
        # thread enqueues on the stream itself drains it first
        self._launcher = ops.Launcher(self._dev_index, self._stream_h)
        self._pool = None
        # decode-only steps: the attention hints (one query per sequence, at
        # most max_seq_len tokens, which bounds every position) and whether
        # they select the short-decode kernel, which needs no plan
        self._short_decode = not ops.paged_attention_reads_plan(
            self.H, self.Hkv, self.hd, self.block_size, 1, mc.max_seq_len)
        # decode steps with wo inside the attention launch (vl_decode_attention_wo)
        self._fused_wo = (self._short_decode and self._fused_rows and self.Hkv in (1, 2, 4, 8)
                          and mc.d_model <= 512 and fused_wo)

    def __del__(self):
        # the submission thread may still hold launches of this runner's graphs
        launcher = getattr(self, "_launcher", None)
        if launcher is not None:
            try:
                launcher.drain()
                launcher.close()
            except Exception:  # interpreter shutdown: the library may be gone
                pass

    # ------------------------------------------------------------ interface --
    @property
    def vocab_size(self) -> int:
        return self.model_cfg.vocab_size

    @property
    def cache_bytes(self) -> int:
        return (self.cache_k.numel() + self.cache_v.numel()) * self.cache_k.element_size()

    def execute(self, out) -> Tuple[np.ndarray, List[Tuple[int, int]]]:
        with torch.cuda.device(self.device), torch.cuda.stream(self.stream):
            rows, R, one, ge = self._run(out, self._buf, exec_ids=True)
            if ge is not None:
                self._launcher.wait(self._launcher.submit(ge))
            self._logits_host[:R].copy_(self._logits[:R], non_blocking=True)
            self.stream.synchronize()
            if one:
                self._check_step(self._exec_ids_host.numpy())
            return self._logits_host_np[:R].copy(), rows

    def execute_argmax(self, out) -> Tuple[np.ndarray, List[Tuple[int, int]]]:
        """execute() for a batch whose every logits row is consumed by a plain
        argmax (greedy sampling with nothing masked or penalised, and greedy
        draft verification: vllmlite/sampling.py:49,56-57,
        vllmlite/speculative.py:86-100): returns each row's argmax, ties to the
        lowest index as np.argmax, computed on the device, so R int32 values
        cross to the host instead of R x vocab fp32 logits."""
        return self.collect(self.launch_argmax(out))

    def launch_argmax(self, out):
        """The first half of execute_argmax: stages the step, enqueues its
        forward, the argmax and the copy of the ids to the host, and returns
        at once with a handle for collect(). One launched step may be
        outstanding while the next is staged and launched; a token id t < 0 in
        the next step's sequences stands for row -t - 1 of this step's ids
        (resolved on the device by the first layer's embedding gather).
        A step whose graph is captured costs the host its staging and one
        graph launch: the graph holds the record's host-to-device copy, the
        forward and the argmax (which writes the ids to the device buffer the
        next step reads and to the pinned one collect() reads)."""
        k = self._buf
        rows, R, one, ge = self._run(out, k)
        host = self._ids_hosts_np[k]
        done = self._done[k]
        if ge is not None:
            # a captured step: its argmax writes the ids into the pinned buffer,
            # which collect() watches (set negative first: the argmax writes
            # every row once, ids are >= 0), so no event follows the graph
            host[:R] = -1
            ticket, done = self._launcher.submit(ge), None
        else:
            ticket = 0
            ops.hip_check(ops.hip_runtime().hipEventRecord(done.cuda_event, self._stream_h),
                          "hipEventRecord")
        self._buf ^= 1
        # the handle holds its own buffer and event: a later step that grows
        # the buffers replaces them while this copy may still be queued
        return rows, R, host, (done, ticket), one

    def collect(self, handle) -> Tuple[np.ndarray, List[Tuple[int, int]]]:
        """Waits for a launched step; its ids and rows."""
        rows, R, host, (done, ticket), one = handle
        self._launcher.wait(ticket)
        if done is None:
            ops.host_wait_nonneg(host[:R])
        else:
            ops.hip_check(ops.hip_runtime().hipEventSynchronize(done.cuda_event),
                          "hipEventSynchronize")
        if one:
            self._check_step(host)
        return host[:R].copy(), rows

    @staticmethod
    def _check_step(host: np.ndarray) -> None:
        status = int(host[ops.DECODE_STEP_ROWS])
        if status:
            why = {1: "a wait between its phases ran out",
                   2: "its workgroups were not all on one XCD"}.get(status, f"status {status}")
            raise RuntimeError(f"one-launch decode step failed: {why}; its results are invalid "
                               "(construct HipRunner with one_launch_decode=False)")

    def _run(self, out, k: int, exec_ids: bool = False):
        """CoW copies, staging into pinned record k and the forward; leaves
        the logits rows in self._logits[:R] and their argmax in self._ids and
        in pinned buffer k. Returns (rows, R, one, graph): a captured step is
        not launched here but its graph executable returned, for the caller
        to submit (it holds the record's copy, the forward and the argmax);
        anything else is enqueued here, on the runner's stream, once earlier
        submissions have been launched. A decode step that the one-launch
        kernel takes leaves the ids in self._ids and in pinned buffer k (or,
        exec_ids, execute()'s own); `one` says so. Selects the runner's
        device itself: the engine may call from any thread."""
        ops.hip_check(ops.hip_runtime().hipSetDevice(self._dev_index), "hipSetDevice")
        if out.cow:
            self._launcher.drain()
            with torch.cuda.device(self.device), torch.cuda.stream(self.stream):
                self._copy_on_write(out.cow)
        shape, rows, R = self._stage(out, k)
        if (self._step is not None and shape.decode and
                shape.Tb == ops.DECODE_STEP_ROWS and shape.Sb <= ops.DECODE_STEP_ROWS):
            self._launcher.drain()
            with torch.cuda.device(self.device), torch.cuda.stream(self.stream):
                self._meta[:shape.n_ints].copy_(self._meta_hosts[k][:shape.n_ints],
                                                non_blocking=True)
                self._decode_step(shape, self._exec_ids_host if exec_ids else self._ids_hosts[k])
            self.one_launch_steps += 1
            return rows, R, True, None
        key = (shape.Tb, shape.Sb, shape.Rb, shape.decode, k)
        ge = self._graph_exec.get(key)
        if ge is not None:
            return rows, R, False, ge
        self._launcher.drain()
        with torch.cuda.device(self.device), torch.cuda.stream(self.stream):
            self._forward(shape, k)
            if self.use_graphs:
                self._capture(shape, key, k)
        return rows, R, False, None

    def _decode_step(self, s: "_Shape", host: torch.Tensor) -> None:
        """The step as one vl_decode_step launch (rows = sequences)."""
        meta, n = self._meta, ops.DECODE_STEP_ROWS
        host.numpy()[n] = 0  # the launch's status word
        mc = self.model_cfg
        ops.decode_step(self._step, self.w["tok_emb"], self.w["final_norm"], self.w["lm_head_t"],
                        self.cache_k, self.cache_v, meta[s.tok:s.tok + n], meta[s.pos:s.pos + n],
                        meta[s.slot:s.slot + n], meta[s.lens:s.lens + s.Sb],
                        meta[s.bt:s.bt + s.Sb * s.W].view(s.Sb, s.W), self._ids, self.cos,
                        self.sin, self.H, self.Hkv, self.block_size, mc.max_seq_len, self.scale,
                        1e-5, self._x, self._q, self._attn, self._act, self._logits, self._ids,
                        host)

    # -------------------------------------------------------------- staging --
    def _ensure_capacity(self, T: int, W: int) -> None:
        if T <= self._cap_T and W <= self.W:
            return
        cap = _bucket(max(T, self._cap_T), 64)
        self.W = max(self.W, W)
        self._graphs.clear()
        self._graph_exec.clear()
        self._pool = None
        old_ids = getattr(self, "_ids", None)
        mc, dev = self.model_cfg, self.device
        H, Hkv, hd = self.H, self.Hkv, self.hd
        f32 = dict(dtype=torch.float32, device=dev)
        n_ints = _Shape(cap, cap, cap, self.W).n_ints
        self._meta = torch.zeros(n_ints, dtype=torch.int32, device=dev)
        # two pinned records: a step may be staged while the copy of the one
        # before is still queued behind the device
        self._meta_hosts = [torch.zeros(n_ints, dtype=torch.int32, pin_memory=True)
                            for _ in range(2)]
        self._meta_nps = [m.numpy() for m in self._meta_hosts]
        self._stager.reset()
        self._x = torch.zeros(cap, mc.d_model, **f32)
        self._h = torch.zeros(cap, mc.d_model, **f32)
        self._delta = torch.zeros(cap, mc.d_model, **f32)
        self._qkv = torch.zeros(cap, (H + 2 * Hkv) * hd, **f32)
        self._q = torch.zeros(cap, H, hd, **f32)
        self._attn = torch.zeros(cap, H, hd, **f32)
        self._gu = torch.zeros(cap, 2 * mc.d_ff, **f32)
        self._act = torch.zeros(cap, mc.d_ff, **f32)
        # decode steps: wo's product as one partial row per (sequence, KV head)
        self._parts = torch.zeros(cap, self.Hkv, mc.d_model, **f32)
        self._hsel = torch.zeros(cap, mc.d_model, **f32)
        self._logits = torch.zeros(cap, mc.vocab_size, **f32)
        self._logits_host = torch.zeros(cap, mc.vocab_size, dtype=torch.float32, pin_memory=True)
        self._logits_host_np = self._logits_host.numpy()
        self._ids = torch.zeros(cap, dtype=torch.int32, device=dev)
        # the lm_head launch's argmax keys and arrival count (left zero by each launch)
        self._am_scratch = torch.zeros(cap + 1, dtype=torch.int64, device=dev)
        if old_ids is not None:  # a launched step's ids, still to be read by the next
            self._ids[:old_ids.numel()].copy_(old_ids)
        self._ids_hosts = [torch.zeros(cap, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self._ids_hosts_np = [h.numpy() for h in self._ids_hosts]
        with torch.cuda.device(dev):
            self._done = [torch.cuda.Event() for _ in range(2)]
            for e in self._done:  # created on the runner's device (torch creates events lazily)
                e.record(self.stream)
        ws = ops.paged_attention_workspace_size(cap, cap, H, hd, mc.max_seq_len + 64)
        self._ws = ops.AttentionWorkspace(dev).get(ws)
        self._cap_T = cap

    def _stage(self, out, k: int):
        """The scheduled batch into pinned record k (RecordStager; the forward
        copies it to the device)."""
        mc = self.model_cfg
        for _ in range(2):
            if self._cap_T > 0:
                shape, rows, R, T, width = self._stager.stage(
                    out, self._meta_nps[k], k, self.block_size, mc.max_seq_len, self.W,
                    self._short_decode, self._cap_T)
                if shape is not None:
                    return shape, rows, R
            else:  # no buffers yet
                f = flatten_scheduled(out, self.block_size, mc.max_seq_len)
                T, width = f.T, f.width
            self._launcher.drain()  # the ids of a step in flight are copied over
            with torch.cuda.device(self.device), torch.cuda.stream(self.stream):
                self._ensure_capacity(T, width)
        raise RuntimeError("staging buffers did not grow to the step")

    # -------------------------------------------------------------- forward --
    def _copy_on_write(self, pairs) -> None:
        p = torch.tensor(pairs, dtype=torch.int32).reshape(-1, 2).to(self.device, non_blocking=False)
        ops.copy_blocks(self.cache_k, self.cache_v, p, self.block_size)

    def _forward(self, s: _Shape, k: int) -> None:
        """Pinned record k to the device, the forward, and the argmax of the
        bucket's Rb logits rows into self._ids and pinned buffer k (rows past
        the step's R are the padded rows' and never read)."""
        n = s.n_ints
        if not self._rows_path(s):
            # read from the pinned record by a kernel: as a graph's memcpy node
            # this copy cost ~12 us more per step
            ops.copy_words(self._meta[:n], self._meta_hosts[k][:n])
        if not self._forward_body(s, self._ids_hosts[k], self._meta_hosts[k]):
            ops.argmax_rows(self._logits[:s.Rb], self._ids[:s.Rb], host_out=self._ids_hosts[k])

    def _rows_path(self, s: _Shape) -> bool:
        """Whether shape s runs on the fused projection kernels (whose first
        launch also copies the step's record to the device)."""
        return s.Tb <= min(self.fused_rows_max, ops.LINEAR_ROWS_MAX) and self._fused_rows

    def _forward_body(self, s: _Shape, ids_host: torch.Tensor, rec_host: torch.Tensor) -> bool:
        """The forward of staged shape s into self._logits[:Rb]; True when its
        lm_head launch also wrote the rows' argmax (to self._ids and ids_host).
        rec_host: the pinned record the step was staged into (on the fused
        path layer 0 reads its indices there and copies it to the device)."""
        mc = self.model_cfg
        Tb, Sb, Rb = s.Tb, s.Sb, s.Rb
        meta = self._meta
        tok = meta[s.tok:s.tok + Tb]
        pos = meta[s.pos:s.pos + Tb]
        slot = meta[s.slot:s.slot + Tb]
        lidx = meta[s.lidx:s.lidx + Rb]
        qsl = meta[s.qsl:s.qsl + Sb + 1]
        lens = meta[s.lens:s.lens + Sb]
        bt = meta[s.bt:s.bt + Sb * s.W].view(Sb, s.W)
        x, h, delta = self._x[:Tb], self._h[:Tb], self._delta[:Tb]
        qkv, q, attn = self._qkv[:Tb], self._q[:Tb], self._attn[:Tb]
        gu, act = self._gu[:Tb], self._act[:Tb]
        W = self.w
        if self._rows_path(s):
            self._forward_rows(s, x, q, attn, act, lidx, qsl, lens, bt, ids_host, rec_host)
            return True
        # ids the previous step chose on the device (negative placeholders)
        ops.resolve_tokens(tok, self._ids)
        torch.index_select(W["tok_emb"], 0, tok, out=x)
        ops.rms_norm(h, x, W["layers"][0]["attn_norm"])
        self._plan(s, q, lens, qsl)
        n_layers = mc.n_layers
        for li, L in enumerate(W["layers"]):
            kc, vc = self.cache_k[li], self.cache_v[li]
            torch.mm(h, L["w_qkv"], out=qkv)
            ops.rope_and_cache(qkv, q, kc, vc, pos, slot, self.cos, self.sin, self.H, self.Hkv,
                               self.hd)
            self._attend(s, attn, q, kc, vc, bt, lens, qsl)
            torch.mm(attn.view(Tb, -1), L["wo"], out=delta)
            ops.rms_norm(h, delta, L["ffn_norm"], residual=x)
            torch.mm(h, L["w_gate_up"], out=gu)
            ops.silu_mul(act, gu)
            torch.mm(act, L["w_down"], out=delta)
            nxt = W["layers"][li + 1]["attn_norm"] if li + 1 < n_layers else W["final_norm"]
            ops.rms_norm(h, delta, nxt, residual=x)
        hsel = self._hsel[:Rb]
        torch.index_select(h, 0, lidx, out=hsel)
        torch.mm(hsel, W["lm_head"], out=self._logits[:Rb])
        return False

    def _plan(self, s: _Shape, q, lens, qsl) -> None:
        """The attention plan of the step, shared by its layers (a decode-only
        step's short-decode kernel reads none)."""
        if not s.decode:
            ops.paged_attention_plan(q, self.cache_k[0], lens, qsl, self.block_size, self._ws)

    def _attend(self, s: _Shape, attn, q, kc, vc, bt, lens, qsl) -> None:
        if s.decode:
            ops.paged_attention_run(attn, q, kc, vc, bt, lens, qsl, self.scale, self.block_size,
                                    self._ws, max_query_len=1, min_query_len=1,
                                    max_context_len=self.model_cfg.max_seq_len)
        else:
            ops.paged_attention_run(attn, q, kc, vc, bt, lens, qsl, self.scale, self.block_size,
                                    self._ws)

    def _lm_head(self, s: _Shape, x, lidx, ids_host) -> None:
        """The final RMSNorm and lm_head of the logits rows x[lidx] with their
        argmax (vl_linear_rows_argmax: ids from the same launch)."""
        W, Rb = self.w, s.Rb
        ops.linear_rows_argmax(self._logits[:Rb], x, W["lm_head_t"], W["final_norm"],
                               self._ids[:Rb], self._am_scratch, host_ids=ids_host,
                               row_index=lidx)

    def _layer0_qkv(self, s: _Shape, x_out, q, rec_host) -> None:
        """Layer 0's QKV + RoPE + scatter with the embedding gather (x =
        tok_emb[tok] written to x_out; a placeholder token -(1 + r) is the id
        the previous step chose for its row r, read from the device), its
        token / position / slot indices read from the pinned record, which the
        same launch copies to the device for the step's later launches."""
        W, Tb, n = self.w, s.Tb, s.n_ints
        L = W["layers"][0]
        ops.qkv_rope_cache(q.view(Tb, -1), self.cache_k[0], self.cache_v[0], W["tok_emb"],
                           L["w_qkv_t"], L["attn_norm"], rec_host[s.pos:s.pos + Tb],
                           rec_host[s.slot:s.slot + Tb], self.cos, self.sin, self.H, self.Hkv,
                           self.hd, row_index=rec_host[s.tok:s.tok + Tb], x_out=x_out,
                           prev_ids=self._ids, record=(rec_host[:n], self._meta[:n]))

    def _forward_rows(self, s: _Shape, x, q, attn, act, lidx, qsl, lens, bt, ids_host,
                      rec_host) -> None:
        """The forward by the fused projection kernels (every decode step, and
        prefill steps up to fused_rows_max rows): each projection is one
        launch with its RMSNorm, residual add, SwiGLU or RoPE + K/V scatter
        fused in, so a layer is QKV (+ RoPE + cache), attention, output (+=
        residual), gate|up (SwiGLU), down (+= residual). A decode step of the
        short-decode shape has its output projection inside the attention
        launch (one partial row per KV head) and the residual add in gate|up's
        prologue: four launches per layer."""
        W, Tb, Rb = self.w, s.Tb, s.Rb
        if s.decode and self._fused_wo:
            self._forward_decode_wo(s, x, q, act, lidx, qsl, lens, bt, ids_host, rec_host)
            return
        pos = self._meta[s.pos:s.pos + Tb]
        slot = self._meta[s.slot:s.slot + Tb]
        for li, L in enumerate(W["layers"]):
            kc, vc = self.cache_k[li], self.cache_v[li]
            if li == 0:
                self._layer0_qkv(s, x, q, rec_host)
                self._plan(s, q, lens, qsl)  # reads the record's device copy
            else:
                ops.qkv_rope_cache(q.view(Tb, -1), kc, vc, x, L["w_qkv_t"], L["attn_norm"], pos,
                                   slot, self.cos, self.sin, self.H, self.Hkv, self.hd)
            self._attend(s, attn, q, kc, vc, bt, lens, qsl)
            ops.linear_rows(x, attn.view(Tb, -1), L["wo_t"], mode=ops.LINEAR_ACCUMULATE)
            ops.linear_rows(act, x, L["w_gate_up_t"], L["ffn_norm"], mode=ops.LINEAR_SWIGLU)
            ops.linear_rows(x, act, L["w_down_t"], mode=ops.LINEAR_ACCUMULATE)
        self._lm_head(s, x, lidx, ids_host)

    def _forward_decode_wo(self, s: _Shape, x, q, act, lidx, qsl, lens, bt, ids_host,
                           rec_host) -> None:
        """A decode step in four launches per layer: QKV (+ RoPE + cache);
        attention with wo (vl_decode_attention_wo: parts[s, g] = the outputs
        of KV head g's query heads @ their rows of wo); gate|up over x + the
        parts summed in KV-head order, which also writes that sum, the
        residual, to the other of two row buffers; down added to it there.
        The two buffers swap roles every layer."""
        W, Tb, Rb, Sb = self.w, s.Tb, s.Rb, s.Sb
        xa, xb = x, self._h[:Tb]
        parts = self._parts[:Tb]
        mc = self.model_cfg
        pos = self._meta[s.pos:s.pos + Tb]
        slot = self._meta[s.slot:s.slot + Tb]
        for li, L in enumerate(W["layers"]):
            kc, vc = self.cache_k[li], self.cache_v[li]
            if li == 0:
                self._layer0_qkv(s, xa, q, rec_host)
            else:
                ops.qkv_rope_cache(q.view(Tb, -1), kc, vc, xa, L["w_qkv_t"], L["attn_norm"], pos,
                                   slot, self.cos, self.sin, self.H, self.Hkv, self.hd)
            ops.decode_attention_wo(parts, q, kc, vc, bt, lens, qsl, self.scale,
                                    self.block_size, L["wo"], mc.max_seq_len)
            ops.linear_rows_parts(act, xa, parts, L["w_gate_up_t"], L["ffn_norm"], x_out=xb)
            ops.linear_rows(xb, act, L["w_down_t"], mode=ops.LINEAR_ACCUMULATE)
            xa, xb = xb, xa
        self._lm_head(s, xa, lidx, ids_host)

    def _capture(self, s: _Shape, key, k: int) -> None:
        # A garbage collection inside the capture could free device or pinned
        # host memory of unreachable objects (an earlier runner, say); the
        # stream operations such frees perform are illegal while a capture is
        # active and abort the process. Collect first, and keep the collector
        # off until the capture has ended.
        gc.collect()
        gc.disable()
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self._pool, stream=self.stream):
                self._forward(s, k)
        finally:
            gc.enable()
        if self._pool is None:
            self._pool = g.pool()
        self._graphs[key] = g
        self._graph_exec[key] = g.raw_cuda_graph_exec()
