"""Dynamic batching of concurrent requests into model calls.

`Batcher` has the reference gateway's semantics (serving/predict.py:253-330):
the first request of a batch opens a window of `window_s`; the batch runs
when the window closes or `max_batch_size` requests wait, whichever comes
first; requests that queued behind a running batch join the next one at
once; the batch function runs on one dedicated thread, so the event loop
keeps accepting requests; a batch that raises fails only its own requests;
every result carries its batch size, its queueing time and the batch's
inference time in microseconds.

On the GPU a batch is two stages: `launch` stages the inputs and enqueues
the copies and kernels (it returns as soon as the work is queued) and
`finish` waits for the results.  Given both, the batcher keeps up to `depth`
batches in flight: it launches the next batch before it waits for the
previous one, so the host-to-device copy of batch n + 1 overlaps the model's
work on batch n.  With a single `run_batch` function (depth 1) batches never
overlap, as in the reference.
"""

import asyncio
import concurrent.futures
import dataclasses
import time
import typing
from collections.abc import Callable

_Item = typing.TypeVar('_Item')
_Result = typing.TypeVar('_Result')


@dataclasses.dataclass
class Batched(typing.Generic[_Result]):
    """One request's result and where its time went (microseconds)."""

    value: _Result
    batch_size: int
    wait_us: int
    inference_us: int


class Batcher(typing.Generic[_Item, _Result]):
    """Groups concurrent requests into batched model calls.

    Args:
      run_batch: items -> results (one per item, in order); the depth-1 form.
      max_batch_size: largest batch.
      window_s: how long the first request of a batch waits for others.
      launch, finish: the two-stage form instead of `run_batch`:
        launch(items) -> handle queues the batch's work, finish(handle) ->
        results waits for it.  Launches run on one thread, in order, and
        completions on another, in the same order.
      depth: batches in flight in the two-stage form (>= 1).
    """

    def __init__(
        self,
        run_batch: Callable[[list[_Item]], list[_Result]] | None = None,
        max_batch_size: int = 1,
        window_s: float = 0.0,
        *,
        launch: Callable[[list[_Item]], typing.Any] | None = None,
        finish: Callable[[typing.Any], list[_Result]] | None = None,
        depth: int = 1,
    ):
        if max_batch_size < 1 or window_s < 0 or depth < 1:
            raise ValueError('need max_batch_size >= 1, window_s >= 0 and depth >= 1')
        if (run_batch is None) == (launch is None and finish is None):
            raise ValueError('give either run_batch or launch and finish')
        if run_batch is None and (launch is None or finish is None):
            raise ValueError('the two-stage form needs both launch and finish')
        if run_batch is not None:
            launch, finish, depth = (lambda items: run_batch(items)), (lambda results: results), 1
        self._launch = launch
        self._finish = finish
        self._depth = depth
        self._max_batch_size = max_batch_size
        self._window_s = window_s
        self._queue: asyncio.Queue | None = None
        self._task: asyncio.Task | None = None
        # Launches run on one thread and completions on another, so waiting
        # for batch n never holds back the launch of batch n + 1.
        self._launcher = concurrent.futures.ThreadPoolExecutor(max_workers=1, thread_name_prefix='inference')
        self._finisher = concurrent.futures.ThreadPoolExecutor(max_workers=1, thread_name_prefix='completion')

    def start(self) -> None:
        """Starts the batching loop on the running event loop."""
        self._queue = asyncio.Queue()
        self._task = asyncio.get_running_loop().create_task(self._loop())

    async def close(self) -> None:
        if self._task is not None:
            self._task.cancel()
            try:
                await self._task
            except asyncio.CancelledError:
                pass
        self._launcher.shutdown(wait=True)
        self._finisher.shutdown(wait=True)

    async def submit(self, item: _Item) -> Batched[_Result]:
        """Queues `item`; resolves when its batch has run.

        Raises whatever the batch function raised for the item's batch.
        """
        if self._queue is None:
            raise RuntimeError('Batcher.start() was not called')
        future = asyncio.get_running_loop().create_future()
        await self._queue.put((item, future, time.perf_counter()))
        return await future

    async def _collect(self) -> list[tuple]:
        batch = [await self._queue.get()]
        deadline = time.perf_counter() + self._window_s
        while len(batch) < self._max_batch_size:
            try:  # requests that queued behind the previous batch join at once
                batch.append(self._queue.get_nowait())
                continue
            except asyncio.QueueEmpty:
                pass
            remaining = deadline - time.perf_counter()
            if remaining <= 0:
                break
            try:
                batch.append(await asyncio.wait_for(self._queue.get(), remaining))
            except asyncio.TimeoutError:
                break
        return batch

    @staticmethod
    def _fail(batch, error: BaseException) -> None:
        for _, future, _ in batch:
            if not future.done():
                future.set_exception(error)

    async def _complete(self, batch, handle, started: float) -> None:
        loop = asyncio.get_running_loop()
        try:
            results = await loop.run_in_executor(self._finisher, self._finish, handle)
            if len(results) != len(batch):
                raise RuntimeError(f'the batch function returned {len(results)} results '
                                   f'for {len(batch)} requests')
        except Exception as e:  # pylint: disable=broad-except
            # Isolation point: the error belongs to this batch's callers, and
            # the loop keeps serving later batches.
            self._fail(batch, e)
            return
        inference_us = int((time.perf_counter() - started) * 1e6)
        for (_, future, queued), result in zip(batch, results):
            if not future.done():
                future.set_result(Batched(result, len(batch), int((started - queued) * 1e6), inference_us))

    async def _completer(self, launched: asyncio.Queue, slots: asyncio.Semaphore) -> None:
        # Batches complete in launch order; each frees its pipeline slot.
        while True:
            batch, handle, started = await launched.get()
            try:
                await self._complete(batch, handle, started)
            finally:
                slots.release()

    async def _loop(self) -> None:
        loop = asyncio.get_running_loop()
        slots = asyncio.Semaphore(self._depth)
        launched: asyncio.Queue = asyncio.Queue()
        completer = loop.create_task(self._completer(launched, slots))
        try:
            while True:
                # A slot is free once the batch `depth` places back has
                # completed; requests queue meanwhile and join the next batch.
                await slots.acquire()
                batch = await self._collect()
                batch = [entry for entry in batch if not entry[1].cancelled()]
                if not batch:
                    slots.release()
                    continue
                started = time.perf_counter()
                try:
                    handle = await loop.run_in_executor(self._launcher, self._launch, [b[0] for b in batch])
                except Exception as e:  # pylint: disable=broad-except
                    self._fail(batch, e)
                    slots.release()
                    continue
                await launched.put((batch, handle, started))
        finally:
            completer.cancel()
            try:
                await completer
            except asyncio.CancelledError:
                pass
