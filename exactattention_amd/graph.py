"""HIP graph capture and replay of enqueue-only work (libamdhip64 through ctypes).

ea_hip_attention enqueues fixed-grid kernels with no memsets and no host synchronisation, so a
whole step (and the serving layer's cache append around it) can be captured once and replayed:
one graph launch per step instead of a dozen kernel launches. The reference runs its step the
same way, in captured CUDA graphs (scripts/bench_vs_flashinfer.py:79-111).
"""

from __future__ import annotations

import ctypes

P = ctypes.c_void_p
NODE_KERNEL, NODE_MEMCPY, NODE_MEMSET = 0, 1, 2
_CAPTURE_THREAD_LOCAL = 1


def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    h.hipStreamBeginCapture.argtypes = [P, ctypes.c_int]
    h.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
    h.hipGraphGetNodes.argtypes = [P, ctypes.POINTER(P), ctypes.POINTER(ctypes.c_size_t)]
    h.hipGraphNodeGetType.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    h.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, ctypes.c_size_t]
    h.hipGraphLaunch.argtypes = [P, P]
    h.hipGraphExecDestroy.argtypes = [P]
    h.hipGraphDestroy.argtypes = [P]
    h.hipMemcpyAsync.argtypes = [P, P, ctypes.c_size_t, ctypes.c_int, P]
    h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(P), ctypes.c_uint]
    h.hipEventRecord.argtypes = [P, P]
    h.hipEventSynchronize.argtypes = [P]
    h.hipEventDestroy.argtypes = [P]
    return h


_H = None


def hip_rt():
    """libamdhip64 with the argtypes this module uses (loaded once)."""
    global _H
    if _H is None:
        _H = _hip()
    return _H


MEMCPY_H2D = 1
EVENT_DISABLE_TIMING = 2


class HipGraph:
    """A captured stream segment. capture(stream, fn) records everything fn enqueues on `stream`
    (a torch.cuda.Stream, made current inside fn's caller), then replay(stream) relaunches it."""

    def __init__(self):
        self.h = hip_rt()
        self.graph = P()
        self.exec = P()

    def capture(self, stream, fn) -> None:
        s = P(stream.cuda_stream)
        rc = self.h.hipStreamBeginCapture(s, _CAPTURE_THREAD_LOCAL)
        if rc != 0:
            raise RuntimeError(f"hipStreamBeginCapture: {rc}")
        try:
            fn()
        finally:
            rc = self.h.hipStreamEndCapture(s, ctypes.byref(self.graph))
        if rc != 0:
            raise RuntimeError(f"hipStreamEndCapture: {rc}")
        rc = self.h.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0)
        if rc != 0:
            raise RuntimeError(f"hipGraphInstantiate: {rc}")

    def node_types(self) -> list[int]:
        n = ctypes.c_size_t(0)
        if self.h.hipGraphGetNodes(self.graph, None, ctypes.byref(n)) != 0:
            raise RuntimeError("hipGraphGetNodes")
        nodes = (P * n.value)()
        if self.h.hipGraphGetNodes(self.graph, nodes, ctypes.byref(n)) != 0:
            raise RuntimeError("hipGraphGetNodes")
        out = []
        for i in range(n.value):
            t = ctypes.c_int(-1)
            if self.h.hipGraphNodeGetType(nodes[i], ctypes.byref(t)) != 0:
                raise RuntimeError("hipGraphNodeGetType")
            out.append(t.value)
        return out

    def replay(self, stream) -> None:
        rc = self.h.hipGraphLaunch(self.exec, P(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipGraphLaunch: {rc}")

    def close(self) -> None:
        if self.exec:
            self.h.hipGraphExecDestroy(self.exec)
            self.exec = P()
        if self.graph:
            self.h.hipGraphDestroy(self.graph)
            self.graph = P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
