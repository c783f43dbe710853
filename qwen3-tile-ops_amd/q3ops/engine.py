"""Continuous-batching host engine over the device model (tools/engine.py).

The engine's state and decisions live in the host scheduling core of
libq3ops.so (``q3_sched_*`` in include/q3ops.h): the page pool, one record
per request (prompt length, tokens fed, ids generated, limit, state, pages),
batch building, the commit of a batch's ids and the device step.  The
classes below keep the reference's interface (names, fields, argument
meaning) as views of that core, so that a caller of the reference can
switch:

- ``PagePool``  (engine.py:81-115): ``free`` / ``used`` / ``free_pages`` are
  read from the core's free stack; ``alloc_page`` / ``ensure`` / ``release``
  act on it;
- ``Request``   (engine.py:33-59): ``n_fed``, ``pages`` and ``state`` are the
  core record's once a pool or engine has taken the request; ``generated``
  (the ids) and the per-request ``rng`` stay in Python;
- ``Scheduler`` (engine.py:152-200): ``build_batch`` is ``q3_sched_build``;
- ``Sampler``   (engine.py:118-149): host float64 sampling in the reference's
  order of numpy operations, so that a seeded request draws the same ids;
- ``Engine``    (engine.py:203-250): step = build, guest step, sample,
  ``q3_sched_commit``.

``GpuGuest`` is the device side (``q3_sched_run``): prefill chunks and rows
whose logits the host samples run ``q3_forward_chunk`` over the request's own
page table; greedy decode rows of a batch share ``q3_decode_batch`` launches
whose lm_head keeps the argmax on the device (only the id comes back).  A
guest may answer a request with an ``int`` (a token already chosen on the
device) instead of logits; ``Engine.step`` then uses it as the sample, which
is what ``Sampler.sample`` returns for ``temperature <= 0`` (first index of
the maximum, engine.py:121-122).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from enum import Enum
from typing import Callable, Mapping, Sequence, Union

import numpy as np

from ._lib import check, lib

__all__ = ["State", "SamplingParams", "Request", "BatchItem", "Batch", "PagePool",
           "Sampler", "Scheduler", "Engine", "GpuGuest", "make_gpu_engine"]

PREFILL_CHUNK = 32  # rows of one prefill chunk (engine.py:175)


class State(str, Enum):
    """Request life cycle (engine.py:15-19); the core's Q3_REQ_* codes are
    the member positions."""
    WAITING = "waiting"
    PREFILL = "prefill"
    DECODE = "decode"
    FINISHED = "finished"


_STATES = list(State)


@dataclass
class SamplingParams:
    """engine.py:22-30."""
    max_new: int = 16
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    seed: int = 0
    stop_tokens: set = field(default_factory=set)


class SchedReq(C.Structure):
    """q3_sched_req."""
    _fields_ = [("n_prompt", C.c_uint32), ("n_fed", C.c_uint32), ("n_gen", C.c_uint32),
                ("max_new", C.c_uint32), ("state", C.c_int32), ("n_pages", C.c_uint32)]


class SchedItem(C.Structure):
    """q3_sched_item."""
    _fields_ = [("slot", C.c_int32), ("row_start", C.c_uint32), ("rows", C.c_uint32),
                ("pos", C.c_uint32), ("prefill", C.c_int32), ("needs_logits", C.c_int32)]


class _Core:
    """Owner of one q3_sched handle and the Request objects of its records
    (index = slot = admission order in the core)."""

    def __init__(self, num_pages: int, page_tokens: int) -> None:
        h = C.c_void_p()
        check(lib().q3_sched_create(int(num_pages), int(page_tokens), C.byref(h)), "q3_sched_create")
        self.h = h
        self.num_pages = int(num_pages)
        self.page_tokens = int(page_tokens)
        self.reqs: list = []

    def __del__(self) -> None:
        h = getattr(self, "h", None)
        if h is not None and h.value:
            lib().q3_sched_destroy(h)
            self.h = C.c_void_p()

    def bind(self, req: "Request") -> int:
        """Registers req (once) and returns its slot."""
        if req._core is self:
            return req._slot
        if req._core is not None:
            raise ValueError(f"request {req.rid} belongs to another pool")
        if req._local_pages:
            raise ValueError(f"request {req.rid}: pages can only come from the pool")
        slot = C.c_int32()
        check(lib().q3_sched_add(self.h, req.n_prompt, int(req.params.max_new), C.byref(slot)),
              "q3_sched_add")
        req._core, req._slot = self, slot.value
        self.reqs.append(req)
        self.put(req, n_fed=req._local_n_fed, state=req._local_state)
        return slot.value

    def get(self, req: "Request") -> SchedReq:
        r = SchedReq()
        check(lib().q3_sched_get(self.h, req._slot, C.byref(r)), "q3_sched_get")
        return r

    def put(self, req: "Request", **kw) -> None:
        r = self.get(req)
        r.n_prompt = req.n_prompt
        r.max_new = int(req.params.max_new)
        r.n_gen = len(req.generated)
        if "n_fed" in kw:
            r.n_fed = int(kw["n_fed"])
        if "state" in kw:
            r.state = _STATES.index(State(kw["state"]))
        check(lib().q3_sched_set(self.h, req._slot, C.byref(r)), "q3_sched_set")

    def pages(self, req: "Request") -> list:
        n = C.c_uint32()
        check(lib().q3_sched_pages(self.h, req._slot, None, 0, C.byref(n)), "q3_sched_pages")
        buf = (C.c_uint32 * max(n.value, 1))()
        check(lib().q3_sched_pages(self.h, req._slot, buf, n.value, C.byref(n)), "q3_sched_pages")
        return list(buf[:n.value])

    def free_list(self) -> list:
        n = C.c_uint32()
        buf = (C.c_uint32 * max(self.num_pages, 1))()
        check(lib().q3_sched_free_pages(self.h, buf, self.num_pages, C.byref(n)),
              "q3_sched_free_pages")
        return list(buf[:n.value])


class Request:
    """engine.py:33-59.  ``n_fed`` counts the tokens whose K/V are cached;
    ``pages`` is the logical -> physical page table.  Until a pool or an
    engine takes the request, n_fed / pages / state are held here; after
    that they are the core record's."""

    def __init__(self, rid: int, prompt, params: SamplingParams, generated=None, n_fed: int = 0,
                 pages=None, state: State = State.WAITING, rng=None) -> None:
        self.rid = rid
        self.prompt = list(prompt)
        self.params = params
        self.generated = list(generated or [])
        self.rng = rng if rng is not None else np.random.default_rng(params.seed)
        self._core: _Core | None = None
        self._slot = -1
        self._local_n_fed = int(n_fed)
        self._local_pages = list(pages or [])
        self._local_state = State(state)

    def __repr__(self) -> str:
        return (f"Request(rid={self.rid}, n_prompt={self.n_prompt}, n_fed={self.n_fed}, "
                f"generated={self.generated}, pages={self.pages}, state={self.state.value})")

    @property
    def n_fed(self) -> int:
        return self._core.get(self).n_fed if self._core else self._local_n_fed

    @n_fed.setter
    def n_fed(self, v: int) -> None:
        if self._core:
            self._core.put(self, n_fed=v)
        else:
            self._local_n_fed = int(v)

    @property
    def state(self) -> State:
        return _STATES[self._core.get(self).state] if self._core else self._local_state

    @state.setter
    def state(self, v: State) -> None:
        if self._core:
            self._core.put(self, state=v)
        else:
            self._local_state = State(v)

    @property
    def pages(self) -> list:
        return self._core.pages(self) if self._core else list(self._local_pages)

    @property
    def n_prompt(self) -> int:
        return len(self.prompt)

    @property
    def done(self) -> bool:
        return self.state == State.FINISHED

    @property
    def needs_logits(self) -> bool:
        return self.state in (State.PREFILL, State.DECODE)


@dataclass
class BatchItem:
    """One request's rows in a batch (engine.py:62-70); ``pos`` is n_fed when
    the batch was built."""
    req: Request
    row_start: int
    rows: int
    pos: int
    token_ids: list
    prefill: bool
    needs_logits: bool


@dataclass
class Batch:
    items: list
    total_rows: int
    _core: object = field(default=None, repr=False, compare=False)
    _raw: object = field(default=None, repr=False, compare=False)

    @property
    def requests(self) -> list:
        return [it.req for it in self.items]


class PagePool:
    """Physical KV pages shared by all requests (engine.py:81-115), a view of
    the core's free stack: pages are handed out from its top and returned to
    it, so the assignment order equals the reference's."""

    def __init__(self, num_pages: int, page_tokens: int = 32, _core: _Core | None = None) -> None:
        self._core = _core or _Core(num_pages, page_tokens)

    @property
    def num_pages(self) -> int:
        return self._core.num_pages

    @property
    def page_tokens(self) -> int:
        return self._core.page_tokens

    @property
    def free(self) -> list:
        """Free pages, bottom to top (``alloc_page`` takes the last)."""
        return self._core.free_list()

    @property
    def used(self) -> set:
        return set(range(self.num_pages)) - set(self.free)

    @property
    def free_pages(self) -> int:
        return len(self.free)

    def alloc_page(self) -> int | None:
        page = C.c_int32()
        check(lib().q3_sched_alloc_page(self._core.h, -1, C.byref(page)), "q3_sched_alloc_page")
        return None if page.value < 0 else page.value

    def ensure(self, req: Request, n_tokens: int) -> bool:
        """Grows req.pages to cover n_tokens; False when the pool runs dry
        (the pages taken so far stay with the request)."""
        slot = self._core.bind(req)
        ok = C.c_int32()
        check(lib().q3_sched_ensure(self._core.h, slot, int(n_tokens), C.byref(ok)),
              "q3_sched_ensure")
        return bool(ok.value)

    def release(self, req: Request) -> None:
        if req._core is self._core:
            check(lib().q3_sched_release(self._core.h, req._slot), "q3_sched_release")


def _repetition_penalty(x: np.ndarray, generated: Sequence[int], penalty: float) -> None:
    # each distinct generated id once: positive logits shrink, others grow
    # (engine.py:125-130)
    for t in set(generated):
        x[t] = x[t] / penalty if x[t] > 0 else x[t] * penalty


def _top_k_mask(x: np.ndarray, k: int) -> None:
    # keep values >= the k-th largest (ties at the threshold survive)
    # (engine.py:131-133)
    kth = np.partition(x, -k)[-k]
    x[x < kth] = -np.inf


def _top_p_mask(x: np.ndarray, p: float) -> None:
    # nucleus: descending order, softmax relative to the maximum, keep the
    # prefix whose cumulative mass is <= p, always the first
    # (engine.py:134-144)
    order = np.argsort(-x)
    xs = x[order]
    mass = np.exp(xs - xs[0])
    mass /= mass.sum()
    keep = np.cumsum(mass) <= p
    keep[0] = True
    x[order[~keep]] = -np.inf


class Sampler:
    """engine.py:118-149.  Host float64 arithmetic, in the reference's order
    of numpy operations, so that the per-request random stream draws the
    same ids from the same logits."""

    def sample(self, logits: Sequence[float], req: Request) -> int:
        p = req.params
        x = np.array(logits, dtype=np.float64)
        if p.temperature <= 0.0:
            return int(np.argmax(x))
        x /= p.temperature
        if p.repetition_penalty != 1.0:
            _repetition_penalty(x, req.generated, p.repetition_penalty)
        if 0 < p.top_k < x.size:
            _top_k_mask(x, p.top_k)
        if p.top_p < 1.0:
            _top_p_mask(x, p.top_p)
        probs = np.exp(x - np.max(x))
        probs /= probs.sum()
        return int(req.rng.choice(x.size, p=probs))


class Scheduler:
    """engine.py:152-200 over the core: requests in admission order; a
    request still in its prompt contributes one chunk of up to 32 rows, a
    decoding request one row (its last generated id); a request that cannot
    get its pages waits for a later batch."""

    def __init__(self, pool: PagePool, max_rows: int = 32) -> None:
        self.pool = pool
        self.max_rows = int(max_rows)

    @property
    def requests(self) -> list:
        return list(self.pool._core.reqs)

    def add(self, req: Request) -> None:
        self.pool._core.bind(req)

    def finish(self, req: Request) -> None:
        core = self.pool._core
        core.bind(req)
        check(lib().q3_sched_finish(core.h, req._slot), "q3_sched_finish")

    def build_batch(self) -> Batch:
        core = self.pool._core
        cap = max(len(core.reqs), 1)
        raw = (SchedItem * cap)()
        n, rows = C.c_uint32(), C.c_uint32()
        check(lib().q3_sched_build(core.h, self.max_rows, raw, cap, C.byref(n), C.byref(rows)),
              "q3_sched_build")
        items = []
        for it in raw[:n.value]:
            req = core.reqs[it.slot]
            ids = (req.prompt[it.pos:it.pos + it.rows] if it.prefill else [req.generated[-1]])
            items.append(BatchItem(req, it.row_start, it.rows, it.pos, list(ids),
                                   bool(it.prefill), bool(it.needs_logits)))
        return Batch(items, rows.value, core, raw)


GuestResult = Union[Sequence[float], np.ndarray, int]


class Engine:
    """engine.py:203-250: step = build a batch, run the guest step, take one
    id per item with logits (the guest's device id, or the sampler's draw),
    commit them to the core."""

    def __init__(self, guest_step: Callable[[Batch], Mapping[int, GuestResult]],
                 num_pages: int = 256, page_tokens: int = 32, max_rows: int = 32,
                 vocab: int = 151936) -> None:
        self.pool = PagePool(num_pages, page_tokens)
        self.sched = Scheduler(self.pool, max_rows)
        self.sampler = Sampler()
        self.guest_step = guest_step
        self.vocab = vocab
        self.next_rid = 0
        self.steps = 0

    def add_request(self, prompt: Sequence[int], params: SamplingParams | None = None) -> Request:
        req = Request(self.next_rid, list(prompt), params or SamplingParams())
        self.next_rid += 1
        self.sched.add(req)
        return req

    def _pick(self, req: Request, out: GuestResult) -> int:
        if isinstance(out, (int, np.integer)):
            if req.params.temperature > 0.0:
                raise ValueError(f"request {req.rid}: the guest returned an id for a sampled "
                                 "(temperature > 0) request")
            return int(out)
        return self.sampler.sample(out, req)

    def step(self) -> bool:
        """One batch; False when nothing could be scheduled."""
        batch = self.sched.build_batch()
        core = self.pool._core
        if not batch.items:
            check(lib().q3_sched_finish_exhausted(core.h, None), "q3_sched_finish_exhausted")
            return False
        results = self.guest_step(batch)
        stop = (C.c_int32 * len(batch.items))()
        for i, it in enumerate(batch.items):
            if it.needs_logits:
                tok = self._pick(it.req, results[it.req.rid])
                it.req.generated.append(tok)
                stop[i] = int(tok in it.req.params.stop_tokens)
        check(lib().q3_sched_commit(core.h, batch._raw, len(batch.items), stop), "q3_sched_commit")
        self.steps += 1
        return True

    def run(self, max_steps: int = 10000) -> None:
        while self.steps < max_steps and self.step():
            pass

    def outputs(self) -> dict:
        return {r.rid: list(r.generated) for r in self.sched.requests}


class GpuGuest:
    """guest_step on the device model (a ``q3ops.Model``) through
    ``q3_sched_run``:

    - a prefill chunk, or any row whose logits the host sampler needs, runs
      ``q3_forward_chunk(pos, rows)`` after its ids are written to the blob's
      id array at ``pos`` and the request's pages are installed as the page
      table; ``Q3_LM_LOGITS`` returns the last row's logits;
    - greedy decode rows (temperature <= 0) of one batch share
      ``q3_decode_batch`` calls: each row writes its K/V through its own
      page table and its id comes back from the device argmax.
    Every request's result is bit-identical to running it alone: rows of
    different requests share GEMM launches but no arithmetic.
    """

    def __init__(self, model, greedy_on_device: bool = True) -> None:
        self.model = model
        self.vocab = model.layout.vocab
        self.greedy_on_device = greedy_on_device
        self.launches = {"forward_chunk": 0, "decode_batch": 0}

    def __call__(self, batch: Batch) -> dict:
        n = len(batch.items)
        if n == 0:
            return {}
        tokens = np.ascontiguousarray(np.concatenate(
            [np.asarray(it.token_ids, np.int32) for it in batch.items]))
        dev = np.array([int(self.greedy_on_device and not it.prefill
                            and it.req.params.temperature <= 0.0) for it in batch.items], np.int32)
        ids = np.full(n, -1, np.int32)
        need = [i for i, it in enumerate(batch.items) if it.needs_logits and not dev[i]]
        logits = np.zeros((n if need else 1, self.vocab), np.float32)
        check(lib().q3_sched_run(batch._core.h, self.model.handle, batch._raw, n,
                                 tokens.ctypes.data_as(C.c_void_p), dev.ctypes.data_as(C.c_void_p),
                                 ids.ctypes.data_as(C.c_void_p),
                                 logits.ctypes.data_as(C.c_void_p) if need else None,
                                 self.vocab), "q3_sched_run")
        self.launches["forward_chunk"] += int(n - dev.sum())
        self.launches["decode_batch"] += -(-int(dev.sum()) // self.model.layout.seq)
        out: dict = {}
        for i, it in enumerate(batch.items):
            if not it.needs_logits:
                continue
            out[it.req.rid] = int(ids[i]) if dev[i] else logits[i].copy()
        return out


def make_gpu_engine(model, max_rows: int | None = None, greedy_on_device: bool = True) -> Engine:
    """An Engine whose pool is the model's KV pool (max_seq / 32 pages per
    layer) and whose batches run on the device."""
    L = model.layout
    rows = min(PREFILL_CHUNK, L.seq) if max_rows is None else int(max_rows)
    return Engine(GpuGuest(model, greedy_on_device), num_pages=L.max_seq // 32,
                  page_tokens=32, max_rows=rows, vocab=L.vocab)
