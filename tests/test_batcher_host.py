"""Host logic of SpeculativeBatcher (the serving worker's loop, serve/src/batching.rs:
324-445) over a scripted stand-in for the device session: admission order and the
batch limit (:326-341), QueueFull (:117-131), failed admissions (admit_job :471-482),
cancellation of queued and active requests (:363-367), deltas, completion and row
reuse (:405-432).  No GPU: the session is a host object with ContinuousSession's
methods."""
import pytest

import aarambh_hip as A


class ScriptedSession:
    """Each step commits min(2 * rounds, remaining budget) tokens per generating row;
    token t of a request is (seed * 1000 + t).  Prompts of 64 or more ids fail at
    admission like a context-limit error."""

    def __init__(self, capacity):
        self.capacity = capacity
        self.state = [A.ContinuousSession.FREE] * capacity
        self.req = [None] * capacity
        self.log = []

    def admit(self, row, prompt_ids, max_new_tokens, seed=0, prefill_chunk=128):
        if not 0 <= row < self.capacity:
            raise A.ShapeError("row outside the session")
        if self.state[row] != A.ContinuousSession.FREE:
            raise A.ConfigError("row holds a request that has not been retired")
        if len(prompt_ids) >= 64:
            raise A.ShapeError(f"prompt has {len(prompt_ids)} tokens but model max_seq_len is 64")
        self.log.append(("admit", row, seed))
        self.req[row] = {"seed": seed, "budget": max_new_tokens, "tokens": []}
        self.state[row] = A.ContinuousSession.GENERATING if max_new_tokens > 0 else A.ContinuousSession.FINISHED

    def retire(self, row):
        self.log.append(("retire", row))
        self.state[row] = A.ContinuousSession.FREE
        self.req[row] = None

    def rows(self):
        return list(self.state)

    def step(self, rounds=1):
        for b in range(self.capacity):
            if self.state[b] != A.ContinuousSession.GENERATING:
                continue
            r = self.req[b]
            n = min(2 * rounds, r["budget"] - len(r["tokens"]))
            r["tokens"] += [r["seed"] * 1000 + len(r["tokens"]) + i for i in range(n)]
            if len(r["tokens"]) >= r["budget"]:
                self.state[b] = A.ContinuousSession.FINISHED
        return all(s != A.ContinuousSession.GENERATING for s in self.state)

    def results(self, candidates=True):
        out = []
        for b in range(self.capacity):
            r = self.req[b]
            toks = list(r["tokens"]) if r else []
            out.append(A.GenerationOutput(toks, "MaxTokens"))
        return out

    def close(self):
        self.log.append(("close",))


def make(capacity=2, queue=4):
    sess = ScriptedSession(capacity)
    bat = A.SpeculativeBatcher(None, A.BatcherConfig(max_batch_size=capacity, queue_capacity=queue),
                               A.Sampler.greedy_sampler(), session=sess)
    return bat, sess


def collect(events):
    deltas, done, failed = {}, {}, {}
    for ev in events:
        if ev[0] == "delta":
            deltas.setdefault(ev[1], []).extend(ev[2])
        elif ev[0] == "completed":
            done[ev[1]] = ev[2]
        else:
            failed[ev[1]] = ev[2]
    return deltas, done, failed


def test_config_and_queue_limits():
    with pytest.raises(A.ConfigError):
        A.SpeculativeBatcher(None, A.BatcherConfig(max_batch_size=0), A.Sampler.greedy_sampler(),
                             session=ScriptedSession(1))
    with pytest.raises(A.ConfigError):
        A.SpeculativeBatcher(None, A.BatcherConfig(prefill_chunk_size=0), A.Sampler.greedy_sampler(),
                             session=ScriptedSession(1))
    bat, _ = make(capacity=1, queue=2)
    bat.submit(A.GenerationRequest([1], 2))
    bat.submit(A.GenerationRequest([1], 2))
    with pytest.raises(A.QueueFull):
        bat.submit(A.GenerationRequest([1], 2))
    bat.step()  # the first request takes the row, freeing a queue place
    bat.submit(A.GenerationRequest([1], 2))


def test_fifo_admission_batch_limit_and_row_reuse():
    bat, sess = make(capacity=2, queue=8)
    ids = [bat.submit(A.GenerationRequest([1, 2], n, seed=i + 1)) for i, n in enumerate([4, 2, 6])]
    ev = bat.step()
    # two rows: requests 0 and 1 are admitted in submission order, 2 waits
    assert [e for e in sess.log if e[0] == "admit"] == [("admit", 0, 1), ("admit", 1, 2)]
    d, done, _ = collect(ev)
    assert d == {ids[0]: [1000, 1001], ids[1]: [2000, 2001]}
    # request 1 finished in that step: completed and its row retired
    assert set(done) == {ids[1]} and ("retire", 1) in sess.log
    assert sorted(bat.active) == [0] and len(bat.queue) == 1
    ev = bat.step()
    # the waiting request takes the freed row 1
    assert ("admit", 1, 3) in sess.log
    ev += bat.run()
    d, done, failed = collect(ev)
    assert not failed and set(done) == {ids[0], ids[2]}
    assert done[ids[0]].token_ids == [1000, 1001, 1002, 1003]
    assert done[ids[2]].token_ids == [3000 + i for i in range(6)] == d[ids[2]]
    assert not bat.active and not bat.queue and bat.pending() == 0
    assert sess.rows() == [A.ContinuousSession.FREE] * 2


def test_failed_admission_takes_no_row():
    bat, sess = make(capacity=1)
    bad = bat.submit(A.GenerationRequest(list(range(64)), 4))
    good = bat.submit(A.GenerationRequest([5], 2, seed=7))
    d, done, failed = collect(bat.step())
    assert set(failed) == {bad} and "max_seq_len" in failed[bad]
    # the next queued request was admitted in the same step, into the row the failure left free
    assert ("admit", 0, 7) in sess.log and done[good].token_ids == [7000, 7001]


def test_cancel_queued_and_active():
    bat, sess = make(capacity=1)
    a = bat.submit(A.GenerationRequest([1], 10, seed=1))
    b = bat.submit(A.GenerationRequest([1], 10, seed=2))
    c = bat.submit(A.GenerationRequest([1], 2, seed=3))
    ev = bat.step()
    bat.cancel(b)  # still queued: dropped when reached
    bat.cancel(a)  # active: retired at the next step, its row reused
    ev += bat.run()
    d, done, failed = collect(ev)
    assert set(done) == {c} and not failed
    assert d[a] == [1000, 1001] and b not in d
    assert [e for e in sess.log if e[0] == "admit"] == [("admit", 0, 1), ("admit", 0, 3)]


def test_zero_budget_completes_at_admission():
    bat, _ = make(capacity=1)
    z = bat.submit(A.GenerationRequest([1, 2, 3], 0))
    d, done, _ = collect(bat.step())
    assert done[z].token_ids == [] and z not in d


class FailingSession(ScriptedSession):
    """A ScriptedSession whose step() raises on its `fail_at`-th call (a device error
    or an invalid proposal distribution in the batched rounds)."""

    def __init__(self, capacity, fail_at):
        super().__init__(capacity)
        self.calls = 0
        self.fail_at = fail_at

    def step(self, rounds=1):
        self.calls += 1
        if self.calls == self.fail_at:
            raise A.ConfigError("proposal distribution is invalid (zero mass or does not sum to one)")
        return super().step(rounds)


def test_failed_decode_fails_every_active_request_and_keeps_serving():
    """decode_sessions failing (batching.rs:441-450): every active request is answered
    with a failure and leaves its row; queued requests are served afterwards."""
    sess = FailingSession(2, fail_at=2)
    bat = A.SpeculativeBatcher(None, A.BatcherConfig(max_batch_size=2, queue_capacity=8),
                               A.Sampler.greedy_sampler(), session=sess)
    a = bat.submit(A.GenerationRequest([1], 6, seed=1))
    b = bat.submit(A.GenerationRequest([1], 6, seed=2))
    c = bat.submit(A.GenerationRequest([1], 2, seed=3))
    ev = bat.step()  # both rows commit two tokens each
    ev2 = bat.step()  # the batched decode fails
    d, done, failed = collect(ev2)
    assert set(failed) == {a, b} and "proposal distribution" in failed[a] and not done and not d
    assert not bat.active and ("retire", 0) in sess.log and ("retire", 1) in sess.log
    assert sess.rows() == [A.ContinuousSession.FREE] * 2
    ev3 = bat.run()  # the queued request still runs to completion in a freed row
    d, done, failed = collect(ev + ev2 + ev3)
    assert set(done) == {c} and done[c].token_ids == [3000, 3001]
    assert d[a] == [1000, 1001] and d[b] == [2000, 2001]
    assert not bat.active and not bat.queue
