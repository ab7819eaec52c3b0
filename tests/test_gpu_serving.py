"""GPU tests of the serving dispatcher (engine_amd/csrc/serving.cpp) through the C ABI.

The decode step itself is pinned to the oracle by test_gpu_decode.py; here
the dispatcher's greedy tokens are checked against the oracle's decode step
on the same sequence, and every dispatcher result is compared with direct
decoder calls on separate caches (the reference's serving tests compare with
the batch-1 executor the same way):
  * eager dispatch equals serial prefill + decode steps, token for token;
  * asynchronous submissions (serial prefill rows, all-decode batches as one
    batched step, several submissions in flight) equal direct steps with the
    same member counts;
  * the prefill-chunk lane equals serial prefill (bit for bit here: every
    GEMV of the 3-member chunk takes the wave path);
  * grouped decode of a mixed batch equals the direct batched step of the
    group plus the serial row;
  * release is deferred while a submission uses the state, caches are
    reused, the KV budget and the reference's error cases hold, and the
    dispatcher stays usable after each rejected submission;
  * the adapter (AmdBackend) over the dispatcher produces completion events;
  * the loading-time memory plan;
  * handles destroyed in any order (the context first, or by the cycle
    collector) leave serving working and every destroy safe.
"""
import numpy as np
import pytest

from engine_amd import serving as S

from oracle.qwen3_oracle import OracleQwen3

from .decode_helpers import small_weights
from .gpu_helpers import to_dev

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, hidden=1024, q_heads=8, kv_heads=2, head_dim=128, ffn=4608, vocab=2048,
            rope_base=1.0e6, epsilon=1.0e-6)
CAP = 64
G = S.SamplingParams.greedy()


def print_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    env = {"E": E, "ctx": ctx, "store": E.AmdWeightStore(ctx), "n": [0]}
    env["dec"] = build_decoder(env, small_weights(TINY, 4242), max_members=8)
    return env


def build_decoder(env, w, max_members):
    E = env["E"]
    handles = {}
    for name, val in w.items():
        if isinstance(val, tuple):
            t, k, n, enc = val
            env["n"][0] += 1
            key = f"s{env['n'][0]}"
            env["store"].materialize_quantized(key, [k, n], t, enc)
            handles[name] = env["store"].quantized_tensor(key)
        else:
            handles[name] = to_dev(val)
    layers = [{f: handles[f"blk.{l}.{f}"] for f in
               ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down", "attn_norm",
                "attn_q_norm", "attn_k_norm", "ffn_norm")} for l in range(TINY["layers"])]
    dec = E.AmdQwen3Decode(env["ctx"], E.AmdQwen3Config(**TINY), handles["token_embd"], handles["output"],
                           handles["output_norm"], layers, max_members)
    return dec


def cache(env, cap=CAP):
    return env["E"].AmdKvCache(env["ctx"], env["E"].AmdQwen3Config(**TINY), cap)


class Request:
    """A request's logical side: its state and the next segment."""
    ids = [1000]

    def __init__(self, prompt, cap=CAP):
        Request.ids[0] += 1
        self.rid = Request.ids[0]
        self.state = S.InferenceStateSet(self.rid, kv_tokens=cap)
        self.prompt = list(prompt)
        self.generated = []

    def prefill(self, sampling=G):
        return S.ExecutionSegment(self.rid, S.Phase.PREFILL, len(self.prompt), 0, tuple(self.prompt), sampling)

    def decode(self):
        pos = len(self.prompt) + len(self.generated) - 1
        return S.ExecutionSegment(self.rid, S.Phase.DECODE, 1, pos, (self.generated[-1],), G)


def run(disp, reqs, segs, submission=None):
    """Submits (or eagerly dispatches) one batch, then commits positions."""
    batch = S.ExecutionBatch(tuple(segs))
    states = [r.state for r in reqs]
    if submission is None:
        outs = disp.dispatch_batch(None, batch, None, states)
    else:
        assert disp.submit_batch(submission, None, batch, None, states) is None
        outs = None
        while outs is None:
            outs = disp.poll_batch(submission)
    S.commit_batch(batch, states)
    for r, o in zip(reqs, outs):
        if o.output_token is not None:
            r.generated.append(o.output_token)
    return outs


def direct(env, prompt, steps, cap=CAP):
    """Serial prefill + greedy decode with direct decoder calls."""
    dec, c = env["dec"], cache(env, cap)
    for i, t in enumerate(prompt[:-1]):
        dec.prefill_step(c, t, i)
    toks = [dec.decode_step(c, prompt[-1], len(prompt) - 1)]
    for s in range(steps):
        toks.append(dec.decode_step(c, toks[-1], len(prompt) + s))
    return toks, c


def test_eager_dispatch_equals_direct_steps(env):
    print_case(test="serving_eager")
    disp = S.AmdServingDispatcher(env["dec"], 4)
    r = Request([5, 1500, 77, 2047, 9])
    outs = run(disp, [r], [r.prefill()])
    assert outs[0].output_token is not None and outs[0].elapsed_nanos > 0
    for _ in range(4):
        run(disp, [r], [r.decode()])
    want, _ = direct(env, r.prompt, 4)
    assert r.generated == want
    assert disp.state_position(r.state) == len(r.prompt) + 4
    disp.close()


def test_dispatcher_tokens_match_the_oracle(env):
    """Eager dispatch of a prompt and eight greedy steps, against the oracle's
    decode step (oracle/qwen3_oracle.py) teacher-forced on the dispatcher's
    own tokens: wherever the oracle's top-2 logit margin exceeds four times
    the decoder's 1e-3 normwise bound, the dispatcher picked the oracle's
    token."""
    print_case(test="serving_oracle")
    disp = S.AmdServingDispatcher(env["dec"], 4)
    r = Request([5, 1500, 77, 2047, 9])
    run(disp, [r], [r.prefill()])
    for _ in range(8):
        run(disp, [r], [r.decode()])
    disp.close()
    orc = OracleQwen3(TINY, small_weights(TINY, 4242), CAP)
    for i, t in enumerate(r.prompt[:-1]):
        orc.step(t, i, head=False)
    seq = r.prompt + r.generated
    checked = 0
    for k, got in enumerate(r.generated):
        pos = len(r.prompt) - 1 + k
        ref = orc.step(seq[pos], pos)
        top2 = np.sort(orc.logits.astype(np.float64))[-2:]
        margin = (top2[1] - top2[0]) / np.abs(orc.logits).max()
        if margin > 4e-3:
            assert got == ref, (k, got, ref, margin)
            checked += 1
    assert checked >= 4, checked


def test_async_submissions_equal_direct_steps(env):
    print_case(test="serving_async")
    dec = env["dec"]
    disp = S.AmdServingDispatcher(dec, 8)
    reqs = [Request([1, 2, 3, 4]), Request([500, 600]), Request([7, 8, 9, 10, 11, 12])]
    # prefill rows in one submission (not batchable: run one by one)
    run(disp, reqs, [r.prefill() for r in reqs], submission=1)
    # two submissions in flight before either is polled
    more = [Request([40, 41, 42]), Request([90])]
    for sid, r in zip((2, 3), more):
        disp.submit_batch(sid, None, S.ExecutionBatch((r.prefill(),)), None, [r.state])
    assert disp.pending_submissions() == 2
    for sid, r in zip((3, 2), more[::-1]):
        outs = None
        while outs is None:
            outs = disp.poll_batch(sid)
        S.commit_batch(S.ExecutionBatch((r.prefill(),)), [r.state])
        r.generated.append(outs[0].output_token)
    # all-decode batches run as one batched step
    all_reqs = reqs + more
    for step in range(3):
        run(disp, all_reqs, [r.decode() for r in all_reqs], submission=10 + step)
    # direct: serial prefill + decode per request, then 5-member batched steps
    caches, nxt, pos = [], [], []
    for r in all_reqs:
        c = cache(env)
        for i, t in enumerate(r.prompt[:-1]):
            dec.prefill_step(c, t, i)
        nxt.append(dec.decode_step(c, r.prompt[-1], len(r.prompt) - 1))
        caches.append(c)
        pos.append(len(r.prompt))
    want = [[t] for t in nxt]
    for _ in range(3):
        nxt = dec.decode_step_batch(caches, nxt, pos)
        for m, t in enumerate(nxt):
            want[m].append(t)
        pos = [p + 1 for p in pos]
    assert [r.generated for r in all_reqs] == want
    assert disp.pending_submissions() == 0 and disp.state_count() == 5
    disp.close()


def test_prefill_chunk_lane_equals_serial_prefill(env):
    print_case(test="serving_prefill_chunk")
    prompt = [(53 * i + 11) % TINY["vocab"] for i in range(11)]
    got = []
    for chunk in (0, 3):
        disp = S.AmdServingDispatcher(env["dec"], 4).with_prefill_chunk(chunk)
        r = Request(prompt)
        run(disp, [r], [r.prefill()], submission=1)
        for s in range(3):
            run(disp, [r], [r.decode()], submission=2 + s)
        got.append(r.generated)
        disp.close()
    want, _ = direct(env, prompt, 3)
    assert got[0] == want and got[1] == want
    with pytest.raises(S.BackendError):
        S.AmdServingDispatcher(env["dec"], 4).with_prefill_chunk(1)
    with pytest.raises(S.BackendError):
        S.AmdServingDispatcher(env["dec"], 4).with_prefill_chunk(9)  # the decoder serves 8 members


def test_prompt_prefill_lane_equals_direct_prompt_prefill(env):
    """The prompt-prefill lane (no reference counterpart): a 40-token prompt's
    first 39 tokens through prefill_prompt (chunks of 16: 16 + 16 + 7), the
    last through the output head, then decode steps, as a submission and
    eagerly; equal token for token to direct prefill_prompt + decode_step
    calls. A 10-token prompt (prefix under 16) keeps the serial path: equal
    to direct serial prefill. Bad chunk sizes are rejected."""
    print_case(test="serving_prompt_prefill")
    dec = env["dec"]
    prompt = [(71 * i + 5) % TINY["vocab"] for i in range(40)]
    c = cache(env)
    dec.prefill_prompt(c, prompt[:-1], 0, 16)
    want = [dec.decode_step(c, prompt[-1], len(prompt) - 1)]
    for s in range(3):
        want.append(dec.decode_step(c, want[-1], len(prompt) + s))
    for submission in (1, None):
        disp = S.AmdServingDispatcher(dec, 4).with_prompt_prefill(16)
        r = Request(prompt)
        run(disp, [r], [r.prefill()], submission=submission)
        for s in range(3):
            run(disp, [r], [r.decode()], submission=None if submission is None else 2 + s)
        assert r.generated == want, (submission, r.generated, want)
        disp.close()
    short = [(31 * i + 9) % TINY["vocab"] for i in range(10)]
    disp = S.AmdServingDispatcher(dec, 4).with_prompt_prefill(16)
    r = Request(short)
    run(disp, [r], [r.prefill()], submission=1)
    for s in range(2):
        run(disp, [r], [r.decode()], submission=2 + s)
    want_short, _ = direct(env, short, 2)
    assert r.generated == want_short
    disp.close()
    with pytest.raises(S.BackendError):
        S.AmdServingDispatcher(dec, 4).with_prompt_prefill(8)
    with pytest.raises(S.BackendError):
        S.AmdServingDispatcher(dec, 4).with_prompt_prefill(4096)


def test_grouped_decode_of_a_mixed_batch(env):
    print_case(test="serving_grouped")
    dec = env["dec"]
    disp = S.AmdServingDispatcher(dec, 8).with_grouped_decode(True)
    a, b = Request([3, 4, 5]), Request([6, 7])
    run(disp, [a, b], [a.prefill(), b.prefill()], submission=1)
    c = Request([8, 9, 10, 11])
    # decode a, prefill c, decode b: a and b run as one 2-member step
    run(disp, [a, c, b], [a.decode(), c.prefill(), b.decode()], submission=2)
    ca, cb = cache(env), cache(env)
    ta, _ = direct(env, a.prompt, 0)
    tb, _ = direct(env, b.prompt, 0)
    for cc, p in ((ca, a.prompt), (cb, b.prompt)):
        for i, t in enumerate(p[:-1]):
            dec.prefill_step(cc, t, i)
        dec.decode_step(cc, p[-1], len(p) - 1)
    pair = dec.decode_step_batch([ca, cb], [ta[0], tb[0]], [len(a.prompt), len(b.prompt)])
    tc, _ = direct(env, c.prompt, 0)
    assert a.generated == [ta[0], pair[0]] and b.generated == [tb[0], pair[1]]
    assert c.generated == tc
    disp.close()


def test_release_is_deferred_and_caches_are_reused(env):
    print_case(test="serving_release")
    disp = S.AmdServingDispatcher(env["dec"], 4)
    r = Request([1, 2, 3])
    run(disp, [r], [r.prefill()], submission=1)
    per = S.qwen3_kv_bytes(env["E"].AmdQwen3Config(**TINY), CAP)
    assert disp.state_bytes() == (per, 0)
    disp.submit_batch(2, None, S.ExecutionBatch((r.decode(),)), None, [r.state])
    disp.release_inference_state(r.state)
    assert disp.state_count() == 1  # the pending submission still uses it
    while disp.poll_batch(2) is None:
        pass
    assert disp.state_count() == 0 and disp.state_bytes() == (0, per)
    disp.release_inference_state(r.state)  # idempotent
    s2 = Request([9, 8, 7])
    run(disp, [s2], [s2.prefill()], submission=3)
    assert disp.state_bytes() == (per, 0)  # the kept cache was reused
    want, _ = direct(env, s2.prompt, 0)
    assert s2.generated == want
    disp.close()


def test_rejected_submissions_leave_the_dispatcher_usable(env):
    print_case(test="serving_errors")
    per = S.qwen3_kv_bytes(env["E"].AmdQwen3Config(**TINY), CAP)
    disp = S.AmdServingDispatcher(env["dec"], 1, kv_budget_bytes=per)  # one slot, one state

    def expect(kind, status, fn):
        with pytest.raises(S.BackendError) as e:
            fn()
        assert e.value.kind == kind and e.value.status == status, str(e.value)

    def submit(sid, segs, states):
        return disp.submit_batch(sid, None, S.ExecutionBatch(tuple(segs)), None, states)

    r, q, z = Request([1, 2]), Request([3, 4]), Request([5, 6])
    expect("UnknownSubmission", 40, lambda: disp.poll_batch(77))
    # rejected before any state is materialized
    hot = S.ExecutionSegment(r.rid, S.Phase.PREFILL, 2, 0, (1, 2), S.SamplingParams(0.7))
    expect("Unsupported", 38, lambda: submit(1, [hot], [r.state]))
    spec = S.ExecutionSegment(r.rid, S.Phase.SPEC_DRAFT, 1, 0, (1,), G)
    expect("Unsupported", 38, lambda: submit(1, [spec], [r.state]))
    late = S.InferenceStateSet(5555, kv_tokens=CAP, token_position=3)
    expect("ExecutionFailed", 42, lambda: submit(1, [S.ExecutionSegment(5555, S.Phase.DECODE, 1, 3, (4,), G)],
                                                 [late]))
    assert disp.state_count() == 0
    # two sampling rows against one pinned slot: the first row ran (its state
    # advanced, as the reference's would), the batch is rejected, the slot
    # recycled
    expect("ExecutionFailed", 39, lambda: submit(1, [r.prefill(), q.prefill()], [r.state, q.state]))
    assert disp.pending_submissions() == 0 and disp.state_count() == 1
    disp.release_inference_state(r.state)
    assert disp.state_bytes() == (0, per)
    # q reuses the kept cache; a third state exceeds the budget
    run(disp, [q], [q.prefill()], submission=1)
    assert disp.state_bytes() == (per, 0)
    expect("ExecutionFailed", 37, lambda: submit(2, [z.prefill()], [z.state]))
    # a duplicate pending submission id
    submit(2, [q.decode()], [q.state])
    expect("ExecutionFailed", 39, lambda: submit(2, [q.decode()], [q.state]))
    while disp.poll_batch(2) is None:
        pass
    # a segment that does not start at its state's position
    stale = S.ExecutionSegment(q.rid, S.Phase.DECODE, 1, 0, (1,), G)
    expect("ExecutionFailed", 42, lambda: disp.dispatch_batch(None, S.ExecutionBatch((stale,)), None,
                                                              [S.InferenceStateSet(q.rid, CAP, 0)]))
    want, _ = direct(env, q.prompt, 0)
    assert q.generated == want
    disp.close()


def test_backend_over_the_dispatcher(env):
    print_case(test="serving_backend")
    caps = S.BackendCapabilities("rocm", 0, "rocm", 288 << 30)
    plan = S.ExecutionPlan("qwen3-tiny", "rocm", 0, 1, frozenset((S.Phase.PREFILL, S.Phase.DECODE)))
    backend = S.AmdBackend(caps, S.AmdServingDispatcher(env["dec"], 8))
    reqs = [Request([1, 2, 3]), Request([4, 5])]
    batch = S.ExecutionBatch(tuple(r.prefill() for r in reqs))
    sid = backend.submit(plan, batch, [r.state for r in reqs])
    ev = backend.wait(sid)
    S.commit_batch(batch, [r.state for r in reqs])
    for r, e in zip(reqs, ev.events):
        assert e.request == r.rid and e.phase == S.Phase.PREFILL and e.output_token is not None
        r.generated.append(e.output_token)
    batch = S.ExecutionBatch(tuple(r.decode() for r in reqs))
    ev = backend.wait(backend.submit(plan, batch, [r.state for r in reqs]))
    for r, e in zip(reqs, ev.events):
        r.generated.append(e.output_token)
    for r in reqs:
        want, _ = direct(env, r.prompt, 1)
        assert r.generated == want
    backend.release_inference_state(reqs[0].state)
    backend.dispatcher.close()


def test_memory_plan(env):
    print_case(test="memory_plan")
    cfg = env["E"].AmdQwen3Config(layers=36, hidden=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=12288,
                                  vocab=151936)
    per = S.qwen3_kv_bytes(cfg, 4096)
    plan = S.plan_memory(env["ctx"], per, 4)
    assert plan.reserved_sequence_bytes == 4 * per
    assert plan.weight_budget_bytes == plan.free_before_preparation_bytes - 4 * per - (512 << 20)
    with pytest.raises(S.BackendError) as e:
        S.plan_memory(env["ctx"], per, 4, weight_budget_bytes=plan.weight_budget_bytes + (1 << 30))
    assert e.value.status == 37
    with pytest.raises(S.BackendError) as e:
        S.plan_memory(env["ctx"], 1 << 50, 1)
    assert e.value.status == 37


def test_handles_destroyed_in_any_order(env):
    """The context handle may go first: weights, kernels, the decoder and the
    dispatcher keep its stream and scratch alive (reference-counted in the C
    library), so serving continues and every later destroy is safe. Then the
    same objects are dropped inside a reference cycle and collected, which
    finalizes them in no particular order (as an exit-time collection
    does)."""
    import gc
    print_case(test="destroy_order")
    E = env["E"]
    ctx = E.AmdContext(0, own_stream=True)
    mine = {"E": E, "ctx": ctx, "store": E.AmdWeightStore(ctx), "n": [0]}
    dec = build_decoder(mine, small_weights(TINY, 5), max_members=2)
    disp = S.AmdServingDispatcher(dec, 4)
    r = Request([1, 2, 3])
    run(disp, [r], [r.prefill()], submission=1)
    first = list(r.generated)
    ctx.close()  # the caller's reference goes first
    run(disp, [r], [r.decode()], submission=2)
    run(disp, [r], [r.decode()])
    assert len(r.generated) == len(first) + 2
    disp.close()
    dec.close()
    mine["store"] = None
    # a second set, left to the cycle collector
    ctx2 = E.AmdContext(0, own_stream=True)
    env2 = {"E": E, "ctx": ctx2, "store": E.AmdWeightStore(ctx2), "n": [0]}
    dec2 = build_decoder(env2, small_weights(TINY, 6), max_members=1)
    disp2 = S.AmdServingDispatcher(dec2, 2)
    cycle = [ctx2, env2, dec2, disp2]
    cycle.append(cycle)
    del ctx2, env2, dec2, disp2, cycle
    gc.collect()
    env["ctx"].synchronize()

