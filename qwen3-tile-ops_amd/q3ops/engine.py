"""Continuous-batching host engine over the device model (tools/engine.py).

The reference's engine is a host scaffold: a page pool of 32-token KV pages,
a scheduler that packs prefill chunks (first) and decode rows into one batch
of at most ``max_rows`` rows, and a sampler (greedy, temperature, top-k,
top-p, repetition penalty) driven by a ``guest_step(batch)`` callback that
returns logits per request.  The classes below keep that interface (names,
fields, argument meaning) so that a caller of the reference can switch:

- ``PagePool``   (engine.py:81-115): LIFO free list of physical page ids;
- ``Sampler``    (engine.py:118-149): float64 host sampling, per-request
  ``numpy.random.default_rng(seed)`` stream;
- ``Scheduler``  (engine.py:152-200): admission-ordered batch building;
- ``Engine``     (engine.py:203-250): step / run / outputs.

``GpuGuest`` is the device side: prefill chunks and logits rows run through
``q3_forward_chunk`` with the request's own page table, and greedy decode
rows of a batch share one ``q3_decode_batch`` launch sequence whose lm_head
keeps the argmax on the device (only the id comes back).  A guest may answer
a request with an ``int`` (a token already chosen on the device) instead of
logits; ``Engine.step`` then uses it as the sample, which is what
``Sampler.sample`` returns for ``temperature <= 0`` (first index of the
maximum, engine.py:121-122).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Callable, Mapping, Sequence, Union

import numpy as np

__all__ = ["State", "SamplingParams", "Request", "BatchItem", "Batch", "PagePool",
           "Sampler", "Scheduler", "Engine", "GpuGuest", "make_gpu_engine"]

PREFILL_CHUNK = 32  # rows of one prefill chunk (engine.py:175)


class State(str, Enum):
    """Request life cycle (engine.py:15-19)."""
    WAITING = "waiting"
    PREFILL = "prefill"
    DECODE = "decode"
    FINISHED = "finished"


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


@dataclass
class Request:
    """engine.py:33-59: ``n_fed`` counts the tokens whose K/V are cached;
    ``pages`` is the logical -> physical page table."""
    rid: int
    prompt: list
    params: SamplingParams
    generated: list = field(default_factory=list)
    n_fed: int = 0
    pages: list = field(default_factory=list)
    state: State = State.WAITING
    rng: np.random.Generator | None = None

    def __post_init__(self) -> None:
        self.rng = np.random.default_rng(self.params.seed)

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

    @property
    def requests(self) -> list:
        return [it.req for it in self.items]


class PagePool:
    """Physical KV pages shared by all requests (engine.py:81-115).  Pages
    are handed out from the end of the free list and returned to its end,
    so the assignment order equals the reference's."""

    def __init__(self, num_pages: int, page_tokens: int = 32) -> None:
        self.num_pages = int(num_pages)
        self.page_tokens = int(page_tokens)
        self.free = list(range(self.num_pages))
        self.used: set = set()

    def alloc_page(self) -> int | None:
        if not self.free:
            return None
        page = self.free.pop()
        self.used.add(page)
        return page

    def ensure(self, req: Request, n_tokens: int) -> bool:
        """Grows req.pages to cover n_tokens; False when the pool runs dry
        (the pages taken so far stay with the request)."""
        need = -(-int(n_tokens) // self.page_tokens)
        while len(req.pages) < need:
            page = self.alloc_page()
            if page is None:
                return False
            req.pages.append(page)
        return True

    def release(self, req: Request) -> None:
        for page in req.pages:
            if page in self.used:
                self.used.discard(page)
                self.free.append(page)
        req.pages.clear()

    @property
    def free_pages(self) -> int:
        return len(self.free)


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
    """engine.py:152-200: requests in admission order; a request still in
    its prompt contributes one chunk of up to 32 rows, a decoding request one
    row (its last generated id); a request that cannot get its pages waits
    for a later batch."""

    def __init__(self, pool: PagePool, max_rows: int = 32) -> None:
        self.pool = pool
        self.max_rows = int(max_rows)
        self.requests: list = []

    def add(self, req: Request) -> None:
        self.requests.append(req)

    def finish(self, req: Request) -> None:
        if req.state != State.FINISHED:
            req.state = State.FINISHED
            self.pool.release(req)

    def _prefill_item(self, req: Request, rows: int) -> BatchItem | None:
        chunk = min(PREFILL_CHUNK, req.n_prompt - req.n_fed, self.max_rows - rows)
        if chunk <= 0 or not self.pool.ensure(req, req.n_fed + chunk):
            return None
        end = req.n_fed + chunk
        return BatchItem(req, rows, chunk, req.n_fed, list(req.prompt[req.n_fed:end]),
                         True, end == req.n_prompt)

    def _decode_item(self, req: Request, rows: int) -> BatchItem | None:
        if not req.generated or not self.pool.ensure(req, req.n_fed + 1):
            return None
        return BatchItem(req, rows, 1, req.n_fed, [req.generated[-1]], False, True)

    def build_batch(self) -> Batch:
        items: list = []
        rows = 0
        for req in self.requests:
            if req.done:
                continue
            if req.n_fed < req.n_prompt:
                item = self._prefill_item(req, rows) if rows < self.max_rows else None
            elif len(req.generated) >= req.params.max_new:
                self.finish(req)
                continue
            else:
                item = self._decode_item(req, rows) if rows < self.max_rows else None
            if item is not None:
                items.append(item)
                rows += item.rows
        return Batch(items, rows)


GuestResult = Union[Sequence[float], np.ndarray, int]


class Engine:
    """engine.py:203-250."""

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

    def _finish_exhausted(self) -> None:
        for req in self.sched.requests:
            if (not req.done and req.n_fed >= req.n_prompt
                    and len(req.generated) >= req.params.max_new):
                self.sched.finish(req)

    def step(self) -> bool:
        """One batch; False when nothing could be scheduled."""
        batch = self.sched.build_batch()
        if not batch.items:
            self._finish_exhausted()
            return False
        results = self.guest_step(batch)
        for it in batch.items:
            req = it.req
            req.n_fed += it.rows
            if it.needs_logits:
                out = results[req.rid]
                if isinstance(out, (int, np.integer)):
                    if req.params.temperature > 0.0:
                        raise ValueError(f"request {req.rid}: the guest returned an id for a "
                                         "sampled (temperature > 0) request")
                    tok = int(out)
                else:
                    tok = self.sampler.sample(out, req)
                req.generated.append(tok)
                if tok in req.params.stop_tokens or len(req.generated) >= req.params.max_new:
                    self.sched.finish(req)
                else:
                    req.state = State.DECODE
            elif req.n_fed < req.n_prompt:
                req.state = State.PREFILL
        self.steps += 1
        return True

    def run(self, max_steps: int = 10000) -> None:
        while self.steps < max_steps and self.step():
            pass

    def outputs(self) -> dict:
        return {r.rid: list(r.generated) for r in self.sched.requests}


class GpuGuest:
    """guest_step on the device model (a ``q3ops.Model``).

    - A prefill chunk, or any row whose logits the host sampler needs, runs
      ``q3_forward_chunk(pos, rows)`` after its ids are written to the blob's
      id array at ``pos`` and the request's pages are installed as the page
      table; ``Q3_LM_LOGITS`` returns the last row's logits.
    - Greedy decode rows (temperature <= 0) of one batch go to one
      ``q3_decode_batch`` call: each row writes its K/V through its own page
      table and its id comes back from the device argmax.
    Every request's result is bit-identical to running it alone: rows of
    different requests share GEMM launches but no arithmetic.
    """

    def __init__(self, model, greedy_on_device: bool = True) -> None:
        import torch
        self.model = model
        L = model.layout
        self.page_slots = L.max_seq // 32
        self.max_chunk = L.seq
        self.max_seq = L.max_seq
        self.greedy_on_device = greedy_on_device
        dev = model.blob.device
        self._ids = torch.zeros(L.seq, dtype=torch.int32, device=dev)
        self._out = torch.zeros(L.seq, dtype=torch.int32, device=dev)
        self.launches = {"forward_chunk": 0, "decode_batch": 0}

    def _table(self, req: Request) -> np.ndarray:
        if len(req.pages) > self.page_slots or any(p >= self.page_slots for p in req.pages):
            raise ValueError(f"request {req.rid}: pages {req.pages} exceed the model's pool "
                             f"of {self.page_slots}")
        t = np.zeros(self.page_slots, np.uint16)
        t[:len(req.pages)] = req.pages
        return t

    def _check_rows(self, it: BatchItem) -> None:
        if it.rows > self.max_chunk or it.pos + it.rows > self.max_seq:
            raise ValueError(f"request {it.req.rid}: rows [{it.pos}, {it.pos + it.rows}) "
                             f"exceed chunk {self.max_chunk} / max_seq {self.max_seq}")

    def _run_chunk(self, it: BatchItem, out: dict) -> None:
        import torch
        from .model import LM_LOGITS, LM_NONE
        self._check_rows(it)
        m = self.model
        m.set_page_table(self._table(it.req))
        ids = np.ascontiguousarray(np.asarray(it.token_ids, np.int32))
        o = m.layout["kIDS"] + 4 * it.pos
        m.blob[o:o + 4 * ids.size].copy_(torch.from_numpy(ids.view(np.uint8)))
        m.forward_chunk(it.pos, it.rows, LM_LOGITS if it.needs_logits else LM_NONE,
                        optimize_tail=True)
        self.launches["forward_chunk"] += 1
        if it.needs_logits:
            out[it.req.rid] = m.stage("logits", 1)[0].copy()

    def _run_greedy_rows(self, items: list, out: dict) -> None:
        import torch
        for it in items:
            self._check_rows(it)
        n = len(items)
        ids = np.array([it.token_ids[0] for it in items], np.int32)
        self._ids[:n].copy_(torch.from_numpy(ids))
        pos = np.array([it.pos for it in items], np.int32)
        tables = np.stack([self._table(it.req) for it in items])
        self.model.decode_batch(self._ids, pos, tables, self._out)
        self.launches["decode_batch"] += 1
        got = self._out[:n].cpu().numpy()
        for it, tok in zip(items, got):
            out[it.req.rid] = int(tok)

    def __call__(self, batch: Batch) -> dict:
        out: dict = {}
        greedy_rows = []
        for it in batch.items:
            if (self.greedy_on_device and not it.prefill
                    and it.req.params.temperature <= 0.0):
                greedy_rows.append(it)
            else:
                self._run_chunk(it, out)
        for i in range(0, len(greedy_rows), self.max_chunk):
            self._run_greedy_rows(greedy_rows[i:i + self.max_chunk], out)
        return out


def make_gpu_engine(model, max_rows: int | None = None, greedy_on_device: bool = True) -> Engine:
    """An Engine whose pool is the model's KV pool (max_seq / 32 pages per
    layer) and whose batches run on the device."""
    L = model.layout
    rows = min(PREFILL_CHUNK, L.seq) if max_rows is None else int(max_rows)
    return Engine(GpuGuest(model, greedy_on_device), num_pages=L.max_seq // 32,
                  page_tokens=32, max_rows=rows, vocab=L.vocab)
