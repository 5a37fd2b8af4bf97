"""Dynamic batching of concurrent requests into model calls.

Semantics (the reference gateway's, serving/predict.py:253-330):

* a batch's window opens when the batcher takes its first request and lasts
  `window_s`; the batch closes when the window ends or `max_batch_size`
  requests are waiting, whichever comes first;
* requests that arrived while the previous batch ran are already waiting, so
  they join the next batch at once;
* the model runs off the event loop, so the loop keeps accepting requests;
* a batch whose function raises fails its own requests only;
* every result carries its batch size, how long it waited and how long its
  batch took (microseconds).

Design.  Requests wait in a deque; `submit` appends and sets an
asyncio.Event.  The collecting coroutine sleeps on that event until the
window ends or enough requests wait, then takes up to `max_batch_size` from
the front.

On the GPU a batch is two stages: `launch` stages the inputs and enqueues the
copies and kernels (it returns once the work is queued) and `finish` waits for
the results.  Given both, the batcher keeps up to `depth` batches in flight:
launches run in order on one thread and completions in the same order on
another, so the next batch's host-to-device copy overlaps the model's work on
the previous one.  A single `run_batch` function is the depth-1 form, in
which batches never overlap.

Every submitted request's future is tracked until it is done.  `close`
stops batching and cancels every request not yet resolved: those still
waiting, the batch being launched and the batches in flight (their callers
see asyncio.CancelledError; work already queued on the device finishes,
and its results are dropped).  Requests submitted after `close` are refused.
"""

import asyncio
import collections
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


@dataclasses.dataclass
class _Pending:
    item: typing.Any
    future: asyncio.Future
    arrived: float  # perf_counter() at submit


def _micros(seconds: float) -> int:
    return int(seconds * 1e6)


class Batcher(typing.Generic[_Item, _Result]):
    """Groups concurrent requests into batched model calls.

    Args:
      run_batch: items -> results (one per item, in order); the depth-1 form.
      max_batch_size: largest batch.
      window_s: how long a batch's first request waits for others.
      launch, finish: the two-stage form instead of `run_batch`:
        launch(items) -> handle queues the batch's work and
        finish(handle) -> results waits for it.
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
        two_stage = launch is not None or finish is not None
        if (run_batch is not None) == two_stage:
            raise ValueError('give either run_batch or launch and finish')
        if two_stage and (launch is None or finish is None):
            raise ValueError('the two-stage form needs both launch and finish')
        if run_batch is not None:
            launch, finish, depth = run_batch, None, 1
        self._launch = launch
        self._finish = finish
        self._depth = depth
        self._limit = max_batch_size
        self._window_s = window_s
        self._waiting: collections.deque[_Pending] = collections.deque()
        self._arrival: asyncio.Event | None = None
        self._task: asyncio.Task | None = None
        self._closed = False
        # Futures of every request submitted and not yet done: waiting,
        # being launched or in flight.
        self._unresolved: set[asyncio.Future] = set()
        self._launch_thread = concurrent.futures.ThreadPoolExecutor(max_workers=1, thread_name_prefix='inference')
        self._finish_thread = concurrent.futures.ThreadPoolExecutor(max_workers=1, thread_name_prefix='completion')

    # ------------------------------------------------------------ lifecycle

    def start(self) -> None:
        """Starts batching on the running event loop."""
        self._arrival = asyncio.Event()
        self._task = asyncio.get_running_loop().create_task(self._serve())

    async def close(self) -> None:
        """Stops batching; every request not yet resolved is cancelled."""
        self._closed = True
        task, self._task = self._task, None
        if task is not None:
            task.cancel()
            await asyncio.gather(task, return_exceptions=True)
        self._waiting.clear()
        for future in list(self._unresolved):
            future.cancel()
        self._launch_thread.shutdown(wait=True)
        self._finish_thread.shutdown(wait=True)

    async def submit(self, item: _Item) -> Batched[_Result]:
        """Queues `item` and returns its result once its batch has run.

        Raises what the batch function raised for the item's batch.
        """
        if self._arrival is None:
            raise RuntimeError('Batcher.start() was not called')
        if self._closed:
            raise RuntimeError('the Batcher is closed')
        future = asyncio.get_running_loop().create_future()
        self._unresolved.add(future)
        future.add_done_callback(self._unresolved.discard)
        self._waiting.append(_Pending(item, future, time.perf_counter()))
        self._arrival.set()
        return await future

    # ------------------------------------------------------------ batching

    async def _until_arrival(self, timeout: float | None) -> bool:
        """Sleeps until a request arrives (True) or `timeout` passes (False)."""
        self._arrival.clear()
        try:
            await asyncio.wait_for(self._arrival.wait(), timeout)
        except asyncio.TimeoutError:
            return False
        return True

    async def _next_batch(self) -> list[_Pending]:
        while not self._waiting:
            await self._until_arrival(None)
        closes = time.perf_counter() + self._window_s
        while len(self._waiting) < self._limit:
            left = closes - time.perf_counter()
            if left <= 0 or not await self._until_arrival(left):
                break
        taken = [self._waiting.popleft() for _ in range(min(self._limit, len(self._waiting)))]
        return [p for p in taken if not p.future.cancelled()]

    @staticmethod
    def _reject(batch: list[_Pending], error: BaseException) -> None:
        for pending in batch:
            if not pending.future.done():
                pending.future.set_exception(error)

    def _results_of(self, handle) -> list:
        return handle if self._finish is None else self._finish(handle)

    async def _resolve(self, batch: list[_Pending], handle, began: float) -> None:
        try:
            results = await asyncio.get_running_loop().run_in_executor(self._finish_thread, self._results_of, handle)
            if len(results) != len(batch):
                raise RuntimeError(f'the batch function gave {len(results)} results for {len(batch)} requests')
        except Exception as error:  # pylint: disable=broad-except
            # The error belongs to this batch's callers; later batches run on.
            self._reject(batch, error)
            return
        took = _micros(time.perf_counter() - began)
        for pending, value in zip(batch, results):
            if not pending.future.done():
                pending.future.set_result(Batched(value, len(batch), _micros(began - pending.arrived), took))

    async def _resolver(self, in_flight: asyncio.Queue, slots: asyncio.Semaphore) -> None:
        # Batches resolve in launch order, each freeing its slot.
        while True:
            batch, handle, began = await in_flight.get()
            try:
                await self._resolve(batch, handle, began)
            finally:
                slots.release()

    async def _serve(self) -> None:
        loop = asyncio.get_running_loop()
        slots = asyncio.Semaphore(self._depth)
        in_flight: asyncio.Queue = asyncio.Queue()
        resolver = loop.create_task(self._resolver(in_flight, slots))
        try:
            while True:
                # The slot of the batch `depth` launches back frees when that
                # batch resolves; meanwhile requests wait and join the next one.
                await slots.acquire()
                batch = await self._next_batch()
                if not batch:
                    slots.release()
                    continue
                began = time.perf_counter()
                try:
                    handle = await loop.run_in_executor(self._launch_thread, self._launch, [p.item for p in batch])
                except Exception as error:  # pylint: disable=broad-except
                    self._reject(batch, error)
                    slots.release()
                    continue
                await in_flight.put((batch, handle, began))
        finally:
            resolver.cancel()
            await asyncio.gather(resolver, return_exceptions=True)
