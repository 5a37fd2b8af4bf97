"""Dynamic batching (CPU): the reference gateway's batching semantics
(serving/tests/test_batching.py restated) and the two-stage pipeline that
keeps a batch in flight while the next one is launched."""

import asyncio
import threading
import time

import pytest

from vectra_amd.serving import batcher as batcher_lib


class _Recorder:
    def __init__(self, fail_on=None, delay_s=0.0):
        self.batches = []
        self._fail_on = fail_on
        self._delay_s = delay_s

    def __call__(self, items):
        self.batches.append(list(items))
        time.sleep(self._delay_s)
        if self._fail_on is not None and self._fail_on in items:
            raise ValueError(f'bad item {self._fail_on}')
        return [item * 10 for item in items]


async def _submit_all(batcher, items):
    return await asyncio.gather(*(batcher.submit(i) for i in items), return_exceptions=True)


def _run(batcher, scenario):
    async def main():
        batcher.start()
        try:
            return await scenario(batcher)
        finally:
            await batcher.close()

    return asyncio.run(main())


def test_concurrent_requests_share_batches_up_to_the_limit():
    recorder = _Recorder()
    results = _run(batcher_lib.Batcher(recorder, max_batch_size=4, window_s=0.05),
                   lambda b: _submit_all(b, range(10)))
    assert [r.value for r in results] == [i * 10 for i in range(10)]
    assert [len(b) for b in recorder.batches] == [4, 4, 2]
    assert results[0].batch_size == 4 and results[-1].batch_size == 2
    assert all(r.inference_us >= 0 and r.wait_us >= 0 for r in results)


def test_a_lone_request_waits_at_most_one_window():
    recorder = _Recorder()

    async def scenario(b):
        start = time.perf_counter()
        result = await b.submit(3)
        return result, time.perf_counter() - start

    result, elapsed = _run(batcher_lib.Batcher(recorder, max_batch_size=64, window_s=0.02), scenario)
    assert result.value == 30 and result.batch_size == 1
    assert 0.015 <= elapsed < 0.5
    assert result.wait_us >= 15_000


def test_a_failing_batch_fails_only_its_own_requests():
    recorder = _Recorder(fail_on=2)

    async def scenario(b):
        return await _submit_all(b, [1, 2, 3]), await _submit_all(b, [4, 5])

    first, second = _run(batcher_lib.Batcher(recorder, max_batch_size=3, window_s=0.05), scenario)
    assert all(isinstance(r, ValueError) for r in first)
    assert [r.value for r in second] == [40, 50]


def test_requests_queue_behind_a_running_batch():
    recorder = _Recorder(delay_s=0.05)

    async def scenario(b):
        first = asyncio.ensure_future(b.submit(0))
        await asyncio.sleep(0.01)  # the first batch is now running
        rest = await _submit_all(b, range(1, 6))
        return await first, rest

    first, rest = _run(batcher_lib.Batcher(recorder, max_batch_size=8, window_s=0.0), scenario)
    assert first.batch_size == 1
    assert {r.batch_size for r in rest} == {5}


def test_a_wrong_number_of_results_fails_the_batch():
    results = _run(batcher_lib.Batcher(lambda items: items[:-1], max_batch_size=4, window_s=0.01),
                   lambda b: _submit_all(b, range(3)))
    assert all(isinstance(r, RuntimeError) for r in results)


def test_submit_requires_start():
    b = batcher_lib.Batcher(_Recorder(), max_batch_size=2, window_s=0.0)
    with pytest.raises(RuntimeError):
        asyncio.run(b.submit(1))


@pytest.mark.parametrize('kwargs', [
    {'max_batch_size': 0}, {'window_s': -1.0}, {'depth': 0},
])
def test_invalid_configuration(kwargs):
    with pytest.raises(ValueError):
        batcher_lib.Batcher(_Recorder(), **{'max_batch_size': 2, 'window_s': 0.0, **kwargs})


def test_exactly_one_form_of_batch_function():
    with pytest.raises(ValueError):
        batcher_lib.Batcher(max_batch_size=2)
    with pytest.raises(ValueError):
        batcher_lib.Batcher(_Recorder(), max_batch_size=2, launch=lambda x: x, finish=lambda x: x)
    with pytest.raises(ValueError):
        batcher_lib.Batcher(max_batch_size=2, launch=lambda x: x)


class _TwoStage:
    """launch() records the batch and returns at once; finish() blocks until
    the test releases that batch, so the test sees what is in flight."""

    def __init__(self, fail_launch_on=None, fail_finish_on=None):
        self.log = []
        self.lock = threading.Lock()
        self.release = {}
        self.fail_launch_on = fail_launch_on
        self.fail_finish_on = fail_finish_on

    def launch(self, items):
        with self.lock:
            self.log.append(('launch', tuple(items)))
            self.release[tuple(items)] = threading.Event()
        if self.fail_launch_on in items:
            raise ValueError('launch failed')
        return tuple(items)

    def finish(self, handle):
        self.release[handle].wait(5.0)
        with self.lock:
            self.log.append(('finish', handle))
        if self.fail_finish_on in handle:
            raise KeyError('finish failed')
        return [i * 10 for i in handle]


def test_two_stage_launches_the_next_batch_before_the_previous_finishes():
    stages = _TwoStage()

    async def scenario(b):
        first = asyncio.ensure_future(_submit_all(b, [1, 2]))
        await asyncio.sleep(0.05)
        second = asyncio.ensure_future(_submit_all(b, [3, 4]))
        await asyncio.sleep(0.05)
        launched_before_release = list(stages.log)
        stages.release[(1, 2)].set()
        stages.release[(3, 4)].set()
        return launched_before_release, await first, await second

    before, first, second = _run(
        batcher_lib.Batcher(max_batch_size=2, window_s=0.01, launch=stages.launch, finish=stages.finish, depth=2),
        scenario)
    # Both batches were launched while the first was still unfinished.
    assert before == [('launch', (1, 2)), ('launch', (3, 4))]
    assert [r.value for r in first] == [10, 20] and [r.value for r in second] == [30, 40]
    assert stages.log.index(('finish', (1, 2))) < stages.log.index(('finish', (3, 4)))


def test_two_stage_keeps_at_most_depth_batches_in_flight():
    stages = _TwoStage()

    async def scenario(b):
        pending = [asyncio.ensure_future(_submit_all(b, [i])) for i in range(1, 5)]
        await asyncio.sleep(0.1)
        in_flight = [entry for entry in stages.log if entry[0] == 'launch']
        for key in list(stages.release):
            stages.release[key].set()
        await asyncio.sleep(0.05)
        for key in list(stages.release):  # batches launched after the first releases
            stages.release[key].set()
        results = [await p for p in pending]
        return in_flight, results

    in_flight, results = _run(
        batcher_lib.Batcher(max_batch_size=1, window_s=0.0, launch=stages.launch, finish=stages.finish, depth=2),
        scenario)
    assert len(in_flight) == 2
    assert [r[0].value for r in results] == [10, 20, 30, 40]


def test_two_stage_failures_stay_with_their_batch():
    stages = _TwoStage(fail_launch_on=2, fail_finish_on=5)

    async def scenario(b):
        results = []
        for batch in ([1], [2], [5], [7]):
            task = asyncio.ensure_future(_submit_all(b, batch))
            await asyncio.sleep(0.02)
            for key in list(stages.release):
                stages.release[key].set()
            results.append(await task)
        return results

    results = _run(
        batcher_lib.Batcher(max_batch_size=1, window_s=0.0, launch=stages.launch, finish=stages.finish, depth=2),
        scenario)
    assert results[0][0].value == 10
    assert isinstance(results[1][0], ValueError)
    assert isinstance(results[2][0], KeyError)
    assert results[3][0].value == 70


def test_close_cancels_batches_in_flight_and_being_launched():
    """close() while one batch is in flight (finish blocked) and the next is
    being launched (launch blocked): every caller is released with
    CancelledError instead of waiting forever, and later submissions are
    refused."""
    release = threading.Event()
    launched = []

    def launch(items):
        launched.append(list(items))
        if len(launched) > 1:
            release.wait(5)
        return list(items)

    def finish(handle):
        release.wait(5)
        return [item + 1 for item in handle]

    async def main():
        b = batcher_lib.Batcher(max_batch_size=2, window_s=0.0, launch=launch, finish=finish, depth=2)
        b.start()
        calls = [asyncio.ensure_future(b.submit(i)) for i in range(6)]
        while len(launched) < 2:
            await asyncio.sleep(0.005)
        closing = asyncio.ensure_future(b.close())
        await asyncio.sleep(0.05)
        release.set()  # let the blocked threads return, so shutdown completes
        await asyncio.wait_for(closing, 5)
        outcomes = await asyncio.wait_for(asyncio.gather(*calls, return_exceptions=True), 5)
        with pytest.raises(RuntimeError, match='closed'):
            await b.submit(9)
        return outcomes

    outcomes = asyncio.run(main())
    assert all(isinstance(o, asyncio.CancelledError) for o in outcomes), outcomes
