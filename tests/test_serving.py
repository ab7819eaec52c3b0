"""CPU tests of the serving dispatcher's host rules and the backend adapter.

- Scheduling rules through the C ABI (no device access): the reference's
  chunked-prefix tables (crates/nvidia/src/serving.rs:1150-1200) and
  decode-group cases (serving.rs:1070-1145), plus the batch-level cases the
  grouping code implies.
- Submission ownership and row scattering (engine_amd/csrc/serving_submissions.hpp),
  built with g++ from tests/cpp/serving_rules_test.cpp: the reference's
  submissions.rs tests and nonadjacent_group_slots_return_to_original_positions.
- The adapter (engine_amd.serving.AmdBackend) with the reference's fake
  dispatchers (adapter.rs:314-460): validation before dispatch, missing
  output tokens, release forwarding, whole-batch forwarding, dispatcher-owned
  async completion, terminal async failure.
- KV accounting: 147,456 bytes per token at Qwen3-8B geometry.
"""
import os
import subprocess

import pytest

from engine_amd import serving as S

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_serving_rules_cpp(tmp_path):
    exe = tmp_path / "serving_rules_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "engine_amd", "csrc"),
                    os.path.join(HERE, "cpp", "serving_rules_test.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True)
    assert out.stdout.strip() == "ok"


@pytest.mark.parametrize("count,members,expected", [
    (1, 8, 0), (7, 8, 0), (8, 8, 0), (9, 8, 8), (15, 8, 8), (16, 8, 8), (17, 8, 16), (32, 8, 24), (16, 4, 12),
    (3, 4, 0)])
def test_chunked_prefix_keeps_the_sampling_token_serial(count, members, expected):
    assert S.chunked_prefix_len(count, members, True) == expected


@pytest.mark.parametrize("count,members,expected", [
    (0, 8, 0), (7, 8, 0), (8, 8, 8), (16, 8, 16), (20, 8, 16), (16, 4, 16), (3, 4, 0), (48, 8, 48)])
def test_chunked_prefix_never_exceeds_whole_chunks(count, members, expected):
    assert S.chunked_prefix_len(count, members, False) == expected


def _rows(capacities, prefill=None, sampling=True, positions=1):
    segs, states = [], []
    for i, cap in enumerate(capacities):
        is_prefill = i == prefill
        segs.append(S.ExecutionSegment(i + 1, S.Phase.PREFILL if is_prefill else S.Phase.DECODE, 1, 1,
                                       (7, 7) if is_prefill else (7,),
                                       S.SamplingParams.greedy() if sampling else None))
        states.append(S.InferenceStateSet(100 + i, kv_tokens=cap, token_position=positions))
    return S.ExecutionBatch(tuple(segs)), states


@pytest.mark.parametrize("capacities,prefill,expected", [
    ([4, 4], None, [0, 1]),
    ([4, 5], None, [0]),
    ([4, 5, 4], None, [0, 2]),
    ([4, 4, 4], 1, [0, 2]),
    ([4] * 9, None, list(range(8))),
])
def test_decode_groups_preserve_order_and_kv_compatibility(capacities, prefill, expected):
    batch, states = _rows(capacities, prefill)
    scheduled = [False] * len(capacities)
    assert S.decode_group(batch, states, scheduled, 0, 8) == expected
    for i in expected:
        scheduled[i] = True
    rest = [i for i, done in enumerate(scheduled) if not done]
    if rest:
        group = S.decode_group(batch, states, scheduled, rest[0], 8)
        assert group[0] == rest[0]
        assert all(not scheduled[i] for i in group)


def test_decode_group_ineligible_rows_run_alone():
    # no sampling, no logical position, no KV state: each row is its own group
    for kwargs in (dict(sampling=False), dict(positions=None)):
        batch, states = _rows([4, 4], **kwargs)
        assert S.decode_group(batch, states, [False, False], 0, 8) == [0]
    batch, states = _rows([0, 0])
    assert S.decode_group(batch, states, [False, False], 0, 8) == [0]


def test_qwen3_kv_bytes_per_token():
    from engine_amd import AmdQwen3Config
    cfg = AmdQwen3Config(layers=36, hidden=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936)
    assert S.qwen3_kv_bytes(cfg, 1) == 147_456
    assert S.qwen3_kv_bytes(cfg, 4096) == 147_456 * 4096


# ---------------------------------------------------------------- adapter

class TestDispatcher(S.AmdDispatcher):
    def dispatch(self, plan, segment, weights, state):
        return S.ExecutionOutcome(12)


class BatchAwareDispatcher(S.AmdDispatcher):
    def __init__(self):
        self.batches = self.segments = self.releases = 0

    def dispatch(self, plan, segment, weights, state):
        self.segments += 1
        return S.ExecutionOutcome(99)

    def dispatch_batch(self, plan, batch, weights, states):
        if len(batch) != len(states):
            raise S.BackendError("StateCountMismatch")
        self.batches += 1
        return [S.ExecutionOutcome(7) for _ in batch.segments]

    def release_inference_state(self, state):
        self.releases += 1


class AsyncDispatcher(S.AmdDispatcher):
    def __init__(self):
        self.submits = self.polls = 0
        self.pending = {}

    def dispatch(self, plan, segment, weights, state):
        raise S.BackendError("ExecutionFailed", "async dispatcher should not use synchronous dispatch")

    def submit_batch(self, submission, plan, batch, weights, states):
        self.submits += 1
        self.pending[submission] = len(batch)
        return None

    def poll_batch(self, submission):
        self.polls += 1
        if submission not in self.pending:
            raise S.BackendError("UnknownSubmission")
        return [S.ExecutionOutcome(5) for _ in range(self.pending.pop(submission))]


class FailingAsyncDispatcher(S.AmdDispatcher):
    def __init__(self):
        self.pending = set()

    def submit_batch(self, submission, plan, batch, weights, states):
        self.pending.add(submission)
        return None

    def poll_batch(self, submission):
        if submission not in self.pending:
            raise S.BackendError("UnknownSubmission")
        self.pending.remove(submission)
        raise S.BackendError("ExecutionFailed", "terminal async failure")


CAPS = S.BackendCapabilities("rocm", 0, "rocm", 288 << 30)


def _plan(device=0, backend="rocm", phases=(S.Phase.DECODE,)):
    return S.ExecutionPlan("test-model", backend, device, 1, frozenset(phases))


def _decode_batch(n=1, sampling=None):
    return S.ExecutionBatch(tuple(S.ExecutionSegment(i + 1, S.Phase.DECODE, 1, 0, (3,), sampling)
                                  for i in range(n)))


def test_backend_requires_rocm_capabilities():
    with pytest.raises(S.BackendError) as e:
        S.AmdBackend(S.BackendCapabilities("cuda", 0, "cuda", 1), TestDispatcher())
    assert e.value.kind == "Unsupported"


def test_backend_dispatches_only_after_capability_and_state_validation():
    backend = S.AmdBackend(CAPS, TestDispatcher())
    batch = _decode_batch()
    for plan, states, kind in ((_plan(device=1), [S.InferenceStateSet(1)], "PlanMismatch"),
                               (_plan(backend="other"), [S.InferenceStateSet(1)], "PlanMismatch"),
                               (_plan(phases=(S.Phase.PREFILL,)), [S.InferenceStateSet(1)], "InvalidPlan"),
                               (_plan(), [], "StateCountMismatch"),
                               (_plan(), [S.InferenceStateSet(1, token_position=3)], "StateMismatch"),
                               (_plan(), [S.InferenceStateSet(1, device=2)], "StateMismatch")):
        with pytest.raises(S.BackendError) as e:
            backend.submit(plan, batch, states)
        assert e.value.kind == kind
    sid = backend.submit(_plan(), batch, [S.InferenceStateSet(1, token_position=0)])
    event = backend.wait(sid)
    assert event.events[0].elapsed_nanos == 12 and event.events[0].policy_version == 1


def test_backend_rejects_missing_requested_output_token():
    backend = S.AmdBackend(CAPS, TestDispatcher())
    with pytest.raises(S.BackendError) as e:
        backend.submit(_plan(), _decode_batch(sampling=S.SamplingParams.greedy()), [S.InferenceStateSet(1)])
    assert e.value.kind == "ExecutionFailed"


def test_backend_forwards_state_release_to_the_dispatcher():
    backend = S.AmdBackend(CAPS, BatchAwareDispatcher())
    backend.release_inference_state(S.InferenceStateSet(1))
    assert backend.dispatcher.releases == 1


def test_backend_forwards_the_whole_scheduler_batch_to_the_dispatcher():
    backend = S.AmdBackend(CAPS, BatchAwareDispatcher())
    sid = backend.submit(_plan(), _decode_batch(2), [S.InferenceStateSet(1), S.InferenceStateSet(2)])
    done = backend.wait(sid)
    assert len(done.events) == 2 and all(e.elapsed_nanos == 7 for e in done.events)
    assert backend.dispatcher.batches == 1 and backend.dispatcher.segments == 0


def test_backend_supports_dispatcher_owned_async_completion():
    backend = S.AmdBackend(CAPS, AsyncDispatcher())
    sid = backend.submit(_plan(), _decode_batch(), [S.InferenceStateSet(1)])
    assert backend.dispatcher.submits == 1 and backend.dispatcher.polls == 0
    done = backend.poll(sid)
    assert done.events[0].elapsed_nanos == 5
    assert backend.dispatcher.polls == 1 and not backend.pending


def test_terminal_async_failure_releases_backend_pending_metadata():
    backend = S.AmdBackend(CAPS, FailingAsyncDispatcher())
    sid = backend.submit(_plan(), _decode_batch(), [S.InferenceStateSet(1)])
    assert len(backend.pending) == 1
    with pytest.raises(S.BackendError) as e:
        backend.poll(sid)
    assert e.value.kind == "ExecutionFailed"
    assert not backend.pending and not backend.dispatcher.pending
    with pytest.raises(S.BackendError) as e:
        backend.poll(sid)
    assert e.value.kind == "UnknownSubmission"


def test_default_dispatcher_has_no_async_completion():
    with pytest.raises(S.BackendError) as e:
        TestDispatcher().poll_batch(1)
    assert e.value.kind == "Unsupported"
    with pytest.raises(S.BackendError) as e:
        TestDispatcher().dispatch_batch(_plan(), _decode_batch(2), None, [S.InferenceStateSet(1)])
    assert e.value.kind == "StateCountMismatch"


def test_commit_batch_moves_prefixes_past_segments():
    batch = S.ExecutionBatch((S.ExecutionSegment(1, S.Phase.PREFILL, 5, 0, (1, 2, 3, 4, 5)),
                              S.ExecutionSegment(2, S.Phase.DECODE, 1, 9, (4,))))
    states = [S.InferenceStateSet(1), S.InferenceStateSet(2, token_position=9)]
    S.commit_batch(batch, states)
    assert [s.token_position for s in states] == [5, 10]
