"""Step runner: record the kernel launches of one decode step, replay them as
AQL dispatch packets on an HSA queue of the library's own
(``smx_runner_*`` in include/smx.h).

The graph-replay loop of the reference (src/spark_vllm_ascend/plugin/
spark2_5.py:369-376, one captured graph per decode step) maps onto
``record(model.enqueue_step)`` once and ``replay(n)`` for n steps: the step is
device-driven, so the same packets serve every step.  ``fences`` picks what
the queue does between two kernels: ``"agent"`` is exactly what a HIP graph
does (agent-scope acquire and release at every boundary); ``"acquire"``
drops the release, which every kernel of this library allows because it
writes what a later kernel reads with agent-scope stores and waits for them
before it ends.

Recording launches nothing.  The recorded packets keep raw device pointers,
so every tensor the recorded calls name must stay alive (and in place) for
as long as the runner replays them; ``record`` refuses a function that
allocated device memory while it recorded (a temporary freed afterwards
would leave a dangling pointer in the packets; the allocation count it
checks is the process's, so another thread allocating meanwhile also makes
it refuse).  Only this library's calls are recorded, so ``record`` also
refuses a function that launched anything else -- a torch ``copy_`` or
``fill_`` into a preallocated buffer, another library's kernel -- which no
replay would repeat: the function runs under a HIP graph capture on a side
stream (this thread only), where such a launch becomes a graph node instead
of running, and a capture with any node is refused.  Other threads may
launch meanwhile (on their own streams) but must not synchronise the whole
device while a recording runs: HIP refuses a device-wide synchronisation
while any stream is capturing.
"""
from __future__ import annotations

import ctypes
import warnings

import torch

from . import (RUNNER_FENCES_ACQUIRE_ONLY, RUNNER_FENCES_AGENT, SmxError, call,
               check_code_objects, checked_record, load)
from .build import code_object_paths

FENCES = {"agent": RUNNER_FENCES_AGENT, "acquire": RUNNER_FENCES_ACQUIRE_ONLY}


def _allocations() -> int:
    return int(torch.cuda.memory_stats().get("allocation.all.allocated", 0))


class StepRunner:
    """One HSA queue and one recorded launch sequence, bound to the current
    HIP device.  Not thread-safe; calls must not overlap."""

    def __init__(self) -> None:
        lib = load()
        paths = code_object_paths()
        missing = [str(p) for p in paths if not p.exists()]
        if missing:
            raise RuntimeError(f"device code objects not built: {missing}; run "
                               "__graft_entry__.build()")
        record = checked_record()
        if record is not None:  # the record that vouched for the library vouches for these
            check_code_objects(record, paths)
        arr = (ctypes.c_char_p * len(paths))(*[str(p).encode() for p in paths])
        handle = ctypes.c_void_p()
        call("smx_runner_create", arr, len(paths), ctypes.byref(handle))
        self._lib = lib
        self._h = handle
        self._ready = False

    # ------------------------------------------------------------- recording
    def record(self, fn) -> int:
        """Record the launches fn() makes through this library; returns the
        number of packets.  Nothing runs on the GPU meanwhile: fn runs under
        a graph capture of this thread's launches on a side stream, and a
        function that launched anything outside the library is refused."""
        if self._h is None:
            raise RuntimeError("the runner is closed")
        self._ready = False
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph(keep_graph=True)  # kept for counting, never instantiated
        with warnings.catch_warnings():
            # an empty capture is the expected outcome
            warnings.filterwarnings("ignore", message=".*Graph is empty.*")
            with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
                before = _allocations()
                call("smx_runner_begin", self._h)
                try:
                    fn()
                except BaseException:
                    self._lib.smx_runner_end(self._h)  # stop recording; the error wins
                    raise
                after = _allocations()
                ended = self._lib.smx_runner_end(self._h)
                end_error = self._lib.smx_last_error().decode() if ended else ""
        nodes = ctypes.c_int64(-1)
        call("smx_graph_num_nodes", ctypes.c_void_p(graph.raw_cuda_graph()), ctypes.byref(nodes))
        del graph
        if ended != 0:
            raise SmxError("smx_runner_end", ended, end_error)
        if after != before:
            raise RuntimeError(
                f"the recorded function allocated device memory {after - before} time(s); "
                "pass preallocated outputs so no recorded pointer can dangle")
        if nodes.value != 0:
            raise RuntimeError(
                f"the recorded function launched {nodes.value} operation(s) outside this "
                "library (a torch op, another library's kernel): no replay would repeat "
                "them; only smx_* calls can be recorded")
        self._ready = True
        return self.num_packets

    @property
    def num_packets(self) -> int:
        n = ctypes.c_int64()
        call("smx_runner_num_packets", self._h, ctypes.byref(n))
        return int(n.value)

    # ---------------------------------------------------------------- replay
    def replay(self, repeats: int = 1, fences: str = "agent", sync: bool = True) -> None:
        """Enqueue the recorded packets `repeats` times and return.  With
        sync, the current device is synchronised first, so the replay sees
        every result of work enqueued on HIP streams before it."""
        if not self._ready:
            raise RuntimeError("nothing recorded")
        if fences not in FENCES:
            raise ValueError(f"fences must be one of {sorted(FENCES)}")
        if sync:
            torch.cuda.synchronize()
        call("smx_runner_replay", self._h, int(repeats), FENCES[fences])

    def set_drain_timeout(self, seconds: float) -> None:
        """How long a replay waits for a free queue slot before it gives up
        and breaks the runner (default 30 s)."""
        call("smx_runner_set_drain_timeout", self._h, float(seconds))

    def wait(self, timeout_s: float = 60.0) -> None:
        """Block until every replay has completed (SmxError after timeout_s)."""
        call("smx_runner_wait", self._h, float(timeout_s))

    def elapsed(self) -> float:
        """Seconds of GPU time of the last (completed) replay: its first
        kernel's start to its last kernel's end."""
        t = ctypes.c_double()
        call("smx_runner_elapsed", self._h, ctypes.byref(t))
        return float(t.value)

    def run(self, repeats: int = 1, fences: str = "agent", timeout_s: float = 60.0) -> None:
        self.replay(repeats, fences)
        self.wait(timeout_s)

    # --------------------------------------------------------------- cleanup
    def close(self) -> None:
        if self._h is not None:
            self._lib.smx_runner_destroy(self._h)
            self._h = None
            self._ready = False

    def __enter__(self):
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass


__all__ = ["StepRunner", "FENCES", "SmxError"]
