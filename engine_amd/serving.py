"""Serving dispatcher and backend adapter over the C ABI (engine_amd/csrc/serving.cpp).

Mirrors the reference's serving seam above the decode step:
  Phase, SamplingParams, ExecutionSegment, ExecutionBatch, InferenceStateSet,
  ExecutionOutcome, ExecutionEvent, ExecutionBatchEvent, ExecutionPlan,
  BackendCapabilities, BackendError     <- the engine-core values the seam carries
                                           (crates/core/src/{execution,state,backend}.rs), reduced to
                                           the fields the dispatcher and adapter read
  AmdDispatcher                         <- the NvidiaDispatcher trait and its default methods
                                           (crates/nvidia/src/adapter.rs:16-129)
  AmdServingDispatcher                  <- CudaQwen35ServingDispatcher (serving.rs:81-1038), native
  AmdBackend                            <- NvidiaBackend<D> (adapter.rs:131-300)
  plan_memory, qwen3_kv_bytes           <- the loading-time budget (crates/qwen/src/loading.rs:117-132)
The dispatcher's scheduling, state registry, pinned output slots and
completion events live in libribn_amd.so; this module converts the seam's
values to ribn_amd_serving_row arrays and statuses back to BackendError.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass, field
from enum import IntEnum
from typing import Optional

from . import _lib
from .kquant import RANK_DISPATCHER, AmdKernelError, _live, _own

NO_POSITION = 0xFFFFFFFF


class Phase(IntEnum):
    """ExecutionPhase."""
    PREFILL = 0
    DECODE = 1
    SPEC_DRAFT = 2
    SPEC_VERIFY = 3
    ENCODER = 4
    MOE_EXPERT = 5


@dataclass(frozen=True)
class SamplingParams:
    """SamplingParams: only greedy (temperature 0) runs on this path."""
    temperature: float = 0.0

    @staticmethod
    def greedy() -> "SamplingParams":
        return SamplingParams(0.0)


@dataclass(frozen=True)
class ExecutionSegment:
    """One request's share of a scheduler batch: `tokens` is the prompt slice of
    a prefill or the one decode token; `sampling` present = the row returns a
    token."""
    request: int
    phase: Phase
    token_count: int
    state_position: int
    tokens: tuple = ()
    sampling: Optional[SamplingParams] = None

    def requests_sampling(self) -> bool:
        return self.sampling is not None


@dataclass
class InferenceStateSet:
    """A request's logical state: `state_id` is its identity (the registry key),
    `kv_tokens` its KV capacity (0: no KV family), `token_position` the
    committed prefix (None before any), `device` its placement (None: not on
    a device)."""
    state_id: int
    kv_tokens: int = 0
    token_position: Optional[int] = None
    device: Optional[int] = 0


@dataclass(frozen=True)
class ExecutionBatch:
    segments: tuple

    def __post_init__(self):
        if not self.segments:
            raise ValueError("an execution batch holds at least one segment")

    def __len__(self) -> int:
        return len(self.segments)


@dataclass(frozen=True)
class ExecutionOutcome:
    """ExecutionOutcome with ExecutionMetrics.elapsed_nanos."""
    elapsed_nanos: int
    output_token: Optional[int] = None


@dataclass(frozen=True)
class ExecutionEvent:
    request: int
    policy_version: int
    phase: Phase
    token_count: int
    elapsed_nanos: int
    output_token: Optional[int] = None


@dataclass(frozen=True)
class ExecutionBatchEvent:
    events: tuple


@dataclass(frozen=True)
class ExecutionPlan:
    """The plan fields the adapter checks: target backend/device, policy
    version and the phases it was prepared for."""
    model: str
    backend: str
    device: int
    policy_version: int
    phases: frozenset
    weights: object = None


@dataclass(frozen=True)
class BackendCapabilities:
    backend: str
    device: int
    kind: str
    memory_bytes: int
    data_types: tuple = ("f16", "f32")
    quantizations: tuple = ("q4_k", "q5_k", "q6_k")
    graph_capture: bool = True
    streams: bool = True


class BackendError(Exception):
    """BackendError (crates/core/src/backend.rs:188-196): `kind` is the variant
    (Unsupported, PlanMismatch, InvalidPlan, StateCountMismatch, StateMismatch,
    UnknownSubmission, ExecutionFailed); `status` the native status, if any."""

    def __init__(self, kind: str, message: str = "", status: Optional[int] = None):
        self.kind = kind
        self.status = status
        super().__init__(f"{kind}: {message}" if message else kind)


def _backend_error(err: AmdKernelError) -> BackendError:
    kind = {"Unsupported": "Unsupported", "UnknownSubmission": "UnknownSubmission"}.get(err.kind, "ExecutionFailed")
    return BackendError(kind, str(err), err.status)


def _call(status: int):
    if status != 0:
        e = _lib.last_error()
        raise _backend_error(AmdKernelError(status, int(e.expected), int(e.actual),
                                            e.message.decode(errors="replace")))


class AmdDispatcher:
    """The dispatcher seam with the reference trait's default methods: a
    synchronous dispatcher implements dispatch(); asynchronous ones override
    submit_batch()/poll_batch()."""

    def dispatch(self, plan, segment, weights, state) -> ExecutionOutcome:
        raise NotImplementedError

    def release_inference_state(self, state) -> None:
        return None

    def dispatch_batch(self, plan, batch, weights, states) -> list:
        if len(batch) != len(states):
            raise BackendError("StateCountMismatch")
        return [self.dispatch(plan, seg, weights, st) for seg, st in zip(batch.segments, states)]

    def submit_batch(self, submission, plan, batch, weights, states):
        return self.dispatch_batch(plan, batch, weights, states)

    def poll_batch(self, submission):
        raise BackendError("Unsupported", "asynchronous AMD dispatcher completion")


def _rows(batch: ExecutionBatch, states) -> tuple:
    n = len(batch)
    rows = (_lib.ServingRow * n)()
    keep = []
    for i, (seg, st) in enumerate(zip(batch.segments, states)):
        r = rows[i]
        r.request = seg.request
        r.state = st.state_id
        r.phase = int(seg.phase)
        r.state_position = seg.state_position
        if seg.tokens:
            arr = (ctypes.c_uint32 * len(seg.tokens))(*[int(t) for t in seg.tokens])
            keep.append(arr)
            r.tokens = ctypes.cast(arr, ctypes.POINTER(ctypes.c_uint32))
        r.token_count = seg.token_count
        r.requests_sampling = 1 if seg.requests_sampling() else 0
        r.temperature = seg.sampling.temperature if seg.sampling is not None else 0.0
        r.kv_tokens = st.kv_tokens
        r.logical_position = NO_POSITION if st.token_position is None else st.token_position
    return rows, keep


def _outcomes(outs) -> list:
    return [ExecutionOutcome(int(o.elapsed_nanos), int(o.token) if o.has_token else None) for o in outs]


class AmdServingDispatcher(AmdDispatcher):
    """CudaQwen35ServingDispatcher over an AmdQwen3Decode: eager dispatch,
    asynchronous submit/poll with one completion event per submission and
    pinned output slots, the physical state registry and deferred release."""

    def __init__(self, decoder, max_pending_rows: int, kv_budget_bytes: int = 0):
        self.decoder = decoder
        self._lib = _lib.load()
        self.handle = ctypes.c_void_p()
        _call(self._lib.ribn_amd_serving_create(decoder.handle, max_pending_rows, kv_budget_bytes,
                                                ctypes.byref(self.handle)))
        _own(self, RANK_DISPATCHER)
        self._rows = {}

    def with_prefill_chunk(self, members: int) -> "AmdServingDispatcher":
        _call(self._lib.ribn_amd_serving_set_prefill_chunk(self.handle, members))
        return self

    def with_prompt_prefill(self, chunk_tokens: int) -> "AmdServingDispatcher":
        """Prefill prefixes of at least 16 tokens on the prefill matmul
        (AmdQwen3Decode.prefill_prompt) in chunks of `chunk_tokens`; 0 turns
        it off. No reference counterpart; reserves the workspace now."""
        _call(self._lib.ribn_amd_serving_set_prompt_prefill(self.handle, chunk_tokens))
        return self

    def with_grouped_decode(self, enabled: bool) -> "AmdServingDispatcher":
        _call(self._lib.ribn_amd_serving_set_grouped_decode(self.handle, 1 if enabled else 0))
        return self

    def dispatch(self, plan, segment, weights, state) -> ExecutionOutcome:
        return self.dispatch_batch(plan, ExecutionBatch((segment,)), weights, [state])[0]

    def dispatch_batch(self, plan, batch, weights, states) -> list:
        if len(batch) != len(states):
            raise BackendError("StateCountMismatch")
        rows, _keep = _rows(batch, states)
        outs = (_lib.ServingOutcome * len(batch))()
        _call(self._lib.ribn_amd_serving_dispatch_batch(self.handle, rows, len(batch), outs))
        return _outcomes(outs)

    def submit_batch(self, submission: int, plan, batch, weights, states):
        if len(batch) != len(states):
            raise BackendError("StateCountMismatch")
        rows, _keep = _rows(batch, states)
        _call(self._lib.ribn_amd_serving_submit_batch(self.handle, submission, rows, len(batch)))
        self._rows[submission] = len(batch)
        return None

    def poll_batch(self, submission: int):
        n = self._rows.get(submission, 0)
        outs = (_lib.ServingOutcome * max(n, 1))()
        ready = ctypes.c_int32()
        try:
            _call(self._lib.ribn_amd_serving_poll_batch(self.handle, submission, outs, n, ctypes.byref(ready)))
        except BackendError:
            self._rows.pop(submission, None)
            raise
        if not ready.value:
            return None
        del self._rows[submission]
        return _outcomes(outs[:n])

    def release_inference_state(self, state) -> None:
        _call(self._lib.ribn_amd_serving_release_state(self.handle, state.state_id))

    def pending_submissions(self) -> int:
        return int(self._lib.ribn_amd_serving_pending(self.handle))

    def state_count(self) -> int:
        return int(self._lib.ribn_amd_serving_state_count(self.handle))

    def state_bytes(self) -> tuple:
        """(bytes held by live states, bytes kept for reuse)."""
        reusable = ctypes.c_uint64()
        used = self._lib.ribn_amd_serving_state_bytes(self.handle, ctypes.byref(reusable))
        return int(used), int(reusable.value)

    def state_position(self, state) -> int:
        pos = ctypes.c_uint32()
        _call(self._lib.ribn_amd_serving_state_position(self.handle, state.state_id, ctypes.byref(pos)))
        return int(pos.value)

    def close(self):
        if self.handle and _live():
            self._lib.ribn_amd_serving_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def commit_batch(batch: ExecutionBatch, states) -> None:
    """The logical state manager's commit after a completed batch (the
    runtime's job, not the dispatcher's): each state's prefix moves past its
    segment."""
    for seg, st in zip(batch.segments, states):
        st.token_position = seg.state_position + seg.token_count


def completion_event(batch: ExecutionBatch, policy_version: int, outcomes) -> ExecutionBatchEvent:
    """completion_event (adapter.rs:185-228): one outcome per segment, a token
    exactly where sampling was requested."""
    if len(outcomes) != len(batch):
        raise BackendError("ExecutionFailed",
                           f"AMD dispatcher returned {len(outcomes)} outcomes for {len(batch)} request segments")
    events = []
    for seg, out in zip(batch.segments, outcomes):
        if seg.requests_sampling() != (out.output_token is not None):
            raise BackendError("ExecutionFailed",
                               f"AMD dispatcher output-token presence did not match sampling for request {seg.request}")
        if seg.token_count == 0:
            raise BackendError("ExecutionFailed", "segment contained no tokens")
        events.append(ExecutionEvent(seg.request, policy_version, seg.phase, seg.token_count, out.elapsed_nanos,
                                     out.output_token))
    return ExecutionBatchEvent(tuple(events))


@dataclass
class _PendingSubmission:
    batch: ExecutionBatch
    policy_version: int


class AmdBackend:
    """NvidiaBackend<D> (adapter.rs:131-300) for a ROCm device: validates a
    submission, allocates its id, forwards it to the dispatcher and turns
    outcomes into completion events, immediately (synchronous dispatchers)
    or when polled (asynchronous ones)."""

    KIND = "rocm"

    def __init__(self, capabilities: BackendCapabilities, dispatcher: AmdDispatcher):
        if capabilities.kind != self.KIND:
            raise BackendError("Unsupported", "ROCm backend capabilities")
        self._capabilities = capabilities
        self.dispatcher = dispatcher
        self._next = 1
        self.completed = {}
        self.pending = {}

    def capabilities(self) -> BackendCapabilities:
        return self._capabilities

    def release_inference_state(self, state) -> None:
        self.dispatcher.release_inference_state(state)

    def validate_execution(self, plan: ExecutionPlan, batch: ExecutionBatch, states) -> None:
        """ComputeBackend::validate_execution (crates/core/src/backend.rs:223-279)."""
        caps = self._capabilities
        if plan.backend != caps.backend or plan.device != caps.device:
            raise BackendError("PlanMismatch", "execution plan targets a different backend/device")
        for seg in batch.segments:
            if seg.phase not in plan.phases:
                raise BackendError("InvalidPlan", f"phase {seg.phase.name} is not prepared by the plan")
        if len(batch) != len(states):
            raise BackendError("StateCountMismatch")
        for seg, st in zip(batch.segments, states):
            if st.token_position is not None and st.token_position != seg.state_position:
                raise BackendError("StateMismatch", "state is at a different prefix position")
            if st.device is not None and st.device != caps.device:
                raise BackendError("StateMismatch", "state is resident on a different device")

    def _allocate(self) -> int:
        sid = self._next
        self._next += 1
        return sid

    def submit(self, plan: ExecutionPlan, batch: ExecutionBatch, states) -> int:
        self.validate_execution(plan, batch, states)
        sid = self._allocate()
        result = self.dispatcher.submit_batch(sid, plan, batch, plan.weights, states)
        if result is not None:
            self.completed[sid] = completion_event(batch, plan.policy_version, result)
        else:
            self.pending[sid] = _PendingSubmission(batch, plan.policy_version)
        return sid

    def poll(self, submission: int) -> Optional[ExecutionBatchEvent]:
        if submission in self.completed:
            return self.completed.pop(submission)
        if submission not in self.pending:
            raise BackendError("UnknownSubmission", f"backend submission {submission} is unknown")
        try:
            outcomes = self.dispatcher.poll_batch(submission)
        except BackendError:
            self.pending.pop(submission, None)
            raise
        if outcomes is None:
            return None
        pending = self.pending.pop(submission)
        return completion_event(pending.batch, pending.policy_version, outcomes)

    def wait(self, submission: int, timeout_s: float = 600.0) -> ExecutionBatchEvent:
        """Polls until the submission completes (ComputeBackend::wait)."""
        deadline = time.monotonic() + timeout_s
        while True:
            ev = self.poll(submission)
            if ev is not None:
                return ev
            if time.monotonic() > deadline:
                raise BackendError("ExecutionFailed", f"submission {submission} did not complete in {timeout_s} s")
            time.sleep(0)


@dataclass(frozen=True)
class MemoryReport:
    free_before_preparation_bytes: int
    weight_budget_bytes: int
    reserved_sequence_bytes: int


def plan_memory(ctx, per_sequence_state_bytes: int, max_sequences: int, continuation_override: int = 0,
                headroom_bytes: int = 512 << 20, weight_budget_bytes: int = 0) -> MemoryReport:
    """The loading-time budget: continuation reserve for max_sequences,
    headroom, and the weight budget that must fit in what remains."""
    out = _lib.MemoryPlan()
    _call(ctx._lib.ribn_amd_plan_memory(ctx.handle, per_sequence_state_bytes, max_sequences, continuation_override,
                                        headroom_bytes, weight_budget_bytes, ctypes.byref(out)))
    return MemoryReport(int(out.free_before_preparation_bytes), int(out.weight_budget_bytes),
                        int(out.reserved_sequence_bytes))


def qwen3_kv_bytes(config, tokens: int) -> int:
    """KvStateSpec::byte_size of a Qwen3 sequence of `tokens` (f16 K and V)."""
    c = config.to_c()
    return int(_lib.load().ribn_amd_qwen3_kv_bytes(ctypes.byref(c), tokens))


def chunked_prefix_len(token_count: int, members: int, requests_sampling: bool) -> int:
    return int(_lib.load().ribn_amd_serving_chunked_prefix_len(token_count, members, 1 if requests_sampling else 0))


def decode_group(batch: ExecutionBatch, states, scheduled, first: int, max_members: int = 64) -> list:
    rows, _keep = _rows(batch, states)
    n = len(batch)
    sched = (ctypes.c_uint8 * n)(*[1 if s else 0 for s in scheduled])
    out = (ctypes.c_size_t * n)()
    k = _lib.load().ribn_amd_serving_decode_group(rows, n, sched, first, max_members, out)
    return [int(out[i]) for i in range(k)]
