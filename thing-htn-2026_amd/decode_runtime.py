"""Host runtime of the decode engine: batch state, step graphs, the speculation policy and the
token pump that turns device steps into the generator's yields.

Everything here is plumbing around the HIP kernels: it owns device buffers (through torch),
records steps into HIP graphs (``torch.cuda.CUDAGraph``) and moves token ids to the host
through pinned memory. It computes nothing itself.

Observable behaviour kept from the reference (``engine/engine.py:1225-1378``): exactly ``N``
yields of ``B`` Python ints, the first from the prompt forward; a decode step is launched
only when it can still contribute a token to some yield (``tests/launch_count.py:57-65``);
speculative verify steps are exact, so the emitted tokens do not depend on the policy.
"""

from __future__ import annotations

import math
import time

import torch

BF16 = torch.bfloat16


class RowGroup:
    """Sequences ``[b0, b1)`` of a batch: the decode kernels run ``M = (b1 - b0) * T`` rows per
    launch, at most 32, so a larger batch is decoded as several groups inside one step."""

    __slots__ = ("index", "b0", "b1", "n", "hist", "pos", "nxt", "kv")

    def __init__(self, index, b0, b1, state):
        self.index, self.b0, self.b1, self.n = index, b0, b1, b1 - b0
        self.hist = state.hist[b0:b1]
        self.pos = state.pos[b0:b1]
        self.nxt = state.nxt[b0:b1]
        self.kv = [(state.arena[l, 0, b0:b1], state.arena[l, 1, b0:b1]) for l in range(state.arena.shape[0])]


class BatchState:
    """Device state of one batch geometry ``(B, cap, k)``.

    * ``arena``: every layer's K and V cache in one allocation ``[L, 2, B, Nkv, cap, D]`` bf16;
      ``kcache(l)`` / ``vcache(l)`` are the ``[B, Nkv, cap, D]`` views the kernels take (the reference's
      per-layer cache layout).
    * ``hist [B, cap]`` int64: prompt and emitted tokens; slot ``cap - 1`` is the dump slot that
      frozen rows write to.
    * ``pos [B]`` int32: tokens held in the cache per sequence.
    * ``marks [2]`` int64: the prompt length and the tokens each sequence must produce; a row
      with ``pos + 1 - marks[0] >= marks[1]`` is frozen (it has all its tokens).
    * ``nxt [B]`` int64: the plain step's output tokens.
    """

    def __init__(self, spec, B, cap, k, device, group_rows):
        self.B, self.cap, self.k = B, cap, k
        self.arena = torch.zeros((spec.L, 2, B, spec.Nkv, cap, spec.D), dtype=BF16, device=device)
        self.hist = torch.zeros((B, cap), dtype=torch.int64, device=device)
        self.pos = torch.zeros((B,), dtype=torch.int32, device=device)
        self.marks = torch.zeros((2,), dtype=torch.int64, device=device)
        self.nxt = torch.zeros((B,), dtype=torch.int64, device=device)
        self.s_mark = self.marks[0:1]
        self.n_mark = self.marks[1:2]
        self.groups = [RowGroup(i, b0, min(B, b0 + group_rows), self)
                       for i, b0 in enumerate(range(0, B, group_rows))]
        self.bufs = {}        # (group index, T) -> StepBuffers
        self.graphs = {}      # T -> StepGraph
        self.certified = {}   # (rows, T) -> verdict
        self.kv_cached = False

    def kcache(self, l):
        return self.arena[l, 0]

    def vcache(self, l):
        return self.arena[l, 1]

    @property
    def kv_bytes(self) -> int:
        return self.arena.numel() * 2

    def open_marks(self):
        """No row is frozen (state used while recording graphs and certifying)."""
        self.marks[0] = 0
        self.marks[1] = 1 << 40


class StepGraph:
    """One decode step recorded as a HIP graph.

    ``issue()`` enqueues the step's kernels and returns its output tensors. Recording runs the
    step once eagerly first (so every kernel is loaded before capture), then captures it; the
    sequence state it touches (``pos``, ``hist``, ``marks``) is saved and restored around both
    runs. The K/V slots and history entries the two runs write lie at positions the prompt
    forward or a later decode step rewrites before anything reads them (every step writes its
    own slots before its attention reads them). ``ms`` is the step time measured on three
    replays after capture, the policy's starting estimate.
    """

    def __init__(self, issue, state, T):
        self.issue, self.state, self.T = issue, state, T
        self.graph = None
        self.outputs = None
        self.ms = None

    def record(self):
        st = self.state
        saved = (st.pos.clone(), st.hist.clone(), st.marks.clone())
        st.open_marks()
        st.pos.zero_()
        self.issue()
        torch.cuda.synchronize()
        st.pos.zero_()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.outputs = self.issue()
        torch.cuda.synchronize()
        self.graph = graph
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.pos.zero_()
        start.record()
        for _ in range(3):
            graph.replay()
        end.record()
        end.synchronize()
        self.ms = start.elapsed_time(end) / 3
        st.pos.copy_(saved[0])
        st.hist.copy_(saved[1])
        st.marks.copy_(saved[2])
        torch.cuda.synchronize()
        return self

    def launch(self):
        self.graph.replay()
        return self.outputs


class SpecPolicy:
    """Chooses between a plain step (one token per row) and a verify step (``k`` drafts).

    Cost model: a verify step gives the slowest unfinished row ``g`` tokens in ``t_v`` ms, a
    plain step one token in ``t_p`` ms, so speculation pays while ``E[g] * t_p > t_v``.
    ``E[g]`` is a running mean with weight ``1/8`` per observation, started at the best case
    (``k + 1``) so that a new call speculates first. Step times start from the graphs' recorded
    times. When speculation stops paying the policy runs plain steps and probes again with
    ``probe_len`` verify steps after a back-off that doubles after every losing probe (from
    ``backoff[0]`` up to ``backoff[1]`` plain steps) and resets when a probe wins.
    ``mode="always"`` speculates on every step that can use it.
    """

    def __init__(self, k, t_plain, t_verify, backoff=(16, 256), probe_len=4, mode="adaptive"):
        self.k = k
        self.t_p = max(float(t_plain), 1e-6)
        self.t_v = max(float(t_verify), 1e-6)
        self.gain = float(k + 1)
        self.backoff_min, self.backoff_max = backoff
        self.backoff = self.backoff_min
        self.probe_len = probe_len
        self.mode = mode
        self.plain_run = 0        # plain steps left before the next probe (0: speculating)
        self.probe_left = 0       # verify steps left in the current probe
        self.verify_steps = 0
        self.verify_gain = 0

    def pays(self) -> bool:
        return self.gain * self.t_p > self.t_v

    def choose(self, tokens_left: int) -> str:
        """Kind of the next step when the slowest row still needs ``tokens_left`` tokens."""
        if self.k == 0 or tokens_left <= 1:
            return "plain"
        if self.mode == "always":
            return "verify"
        if self.plain_run > 0:
            self.plain_run -= 1
            if self.plain_run == 0:
                self.probe_left = self.probe_len
            return "plain"
        if self.probe_left > 0:
            self.probe_left -= 1
        return "verify"

    def observe_verify(self, gain: int):
        """The slowest unfinished row gained ``gain`` tokens from one verify step."""
        self.verify_steps += 1
        self.verify_gain += gain
        self.gain += (gain - self.gain) / 8.0
        if self.mode == "always" or self.plain_run > 0:
            return
        if self.pays():
            if self.probe_left == 0:
                self.backoff = self.backoff_min
        elif self.probe_left == 0:
            self.plain_run = self.backoff
            self.backoff = min(self.backoff * 2, self.backoff_max)

    def observe_time(self, kind: str, ms: float):
        if kind == "plain":
            self.t_p += (ms - self.t_p) / 8.0
        else:
            self.t_v += (ms - self.t_v) / 8.0


class _Ticket:
    __slots__ = ("slot", "kind", "bound", "t0", "t1")

    def __init__(self, slot, kind, bound, timed):
        self.slot, self.kind, self.bound = slot, kind, bound
        self.t0 = torch.cuda.Event(enable_timing=True) if timed else None
        self.t1 = torch.cuda.Event(enable_timing=True) if timed else None


class TokenPump:
    """Drives decode steps and yields one list of ``B`` ints per output position.

    The device runs ahead of the consumer: up to ``depth`` steps are queued, each followed by
    an asynchronous copy of its tokens into its own pinned host slot and an event. The host
    waits only on the oldest step's event, files its tokens per row and yields every position
    that all rows have reached. A step is launched only while the tokens already filed plus
    the most the queued steps can bring stay below ``N`` for the slowest row, so no launched
    step is wasted and none is left running when the last yield happens.

    ``run_plain()`` / ``run_verify()`` enqueue one step and return its output tensors
    (``nxt [B]`` / ``(out_t [T, B], adv [B])``); ``first`` is the prompt forward's token per
    row (on the device).
    """

    def __init__(self, B, N, first, depth, k, run_plain, run_verify, policy, counters):
        self.B, self.N, self.k = B, N, k
        self.first = first
        self.depth = max(1, depth)
        self.run_plain, self.run_verify = run_plain, run_verify
        self.policy = policy
        self.counters = counters
        nslots = self.depth + 1
        self.tok_slots = [torch.zeros((k + 1, B), dtype=torch.int64, pin_memory=True) for _ in range(nslots)]
        self.adv_slots = [torch.zeros((B,), dtype=torch.int64, pin_memory=True) for _ in range(nslots)]
        self.done = [torch.cuda.Event() for _ in range(nslots)]
        self.free = list(range(nslots))

    def _launch(self, kind, stream):
        slot = self.free.pop()
        timed = kind != "first" and self.k > 0
        t = _Ticket(slot, kind, 1 if kind != "verify" else self.k + 1, timed)
        if timed:
            t.t0.record(stream)
        if kind == "first":
            self.tok_slots[slot][0].copy_(self.first, non_blocking=True)
        elif kind == "plain":
            nxt = self.run_plain()
            self.counters["decode"] += 1
            self.tok_slots[slot][0].copy_(nxt, non_blocking=True)
        else:
            out_t, adv = self.run_verify()
            self.counters["decode"] += 1
            self.counters["verify"] += 1
            self.tok_slots[slot].copy_(out_t, non_blocking=True)
            self.adv_slots[slot].copy_(adv, non_blocking=True)
        if timed:
            t.t1.record(stream)
        self.done[slot].record(stream)
        return t

    def __iter__(self):
        B, N = self.B, self.N
        rows = [[] for _ in range(B)]
        emitted = 0
        queue = []
        stream = torch.cuda.current_stream()
        with torch.inference_mode():
            queue.append(self._launch("first", stream))
        in_flight_bound = 1
        while emitted < N:
            slowest = min(len(r) for r in rows)
            with torch.inference_mode():
                while len(queue) < self.depth and slowest + in_flight_bound < N:
                    kind = self.policy.choose(N - slowest - in_flight_bound)
                    t = self._launch(kind, stream)
                    queue.append(t)
                    in_flight_bound += t.bound
            t = queue.pop(0)
            in_flight_bound -= t.bound
            self.done[t.slot].synchronize()
            if t.t0 is not None:
                self.policy.observe_time(t.kind, t.t0.elapsed_time(t.t1))
            if t.kind == "verify":
                toks = self.tok_slots[t.slot].tolist()
                adv = self.adv_slots[t.slot].tolist()
                gains = []
                for b in range(B):
                    a = int(adv[b])
                    unfinished = len(rows[b]) < N
                    rows[b].extend(int(toks[j][b]) for j in range(a))
                    if unfinished:
                        gains.append(a)
                if gains:
                    self.policy.observe_verify(min(gains))
                    self.counters["verify_gain"] += min(gains)
            else:
                for b, tok in enumerate(self.tok_slots[t.slot][0].tolist()):
                    rows[b].append(int(tok))
            self.free.append(t.slot)
            ready = min(len(r) for r in rows)
            while emitted < min(ready, N):
                yield [rows[b][emitted] for b in range(B)]
                emitted += 1


def capacity(S: int, N: int, k: int, round_to: int) -> int:
    """KV / history slots for a prompt of ``S`` tokens and ``N`` outputs with ``k`` drafts per
    verify step: the largest position a row can reach is ``S + N + k - 1`` (its last verify
    step may accept past its last needed token), a frozen row's verify step writes ``k + 1``
    slots from there, and the last slot is the dump slot; rounded up to ``round_to``."""
    need = S + N + 2 * (k + 1) + 2
    return int(math.ceil(need / round_to) * round_to)


def log_time(t0: float) -> str:
    return f"{time.time() - t0:.1f}s"
