"""Program: the port-level runtime contract of the reference (aneforge/_runtime.py:138-248),
over device buffers and a captured kernel sequence instead of an Espresso program.

  set_input(name, arr)   copy a host array into an input port (shape checked)
  execute()              run once, synchronously (the reference's execute is synchronous)
  read_output(name)      a fresh fp16 host copy of an output port
  eval(feed)             set every fed input, execute, read every output
  share_buffer(...)      alias an output onto an input (must precede the first execute): the
                         output is written into the input port's own buffer, so resident state
                         (e.g. a KV cache) is updated in place and never copied; when an op
                         would read the input after the output is written, the output is
                         copied device-to-device into the input after each execute instead
  input_view/output_view the port's device tensor (zero-copy; the reference returns host
                         views of ANE-visible memory)
  release()              drop buffers and the captured graph"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _hip


class Program:
    def __init__(self, inputs: dict, outputs: dict, plan, buffers: dict):
        """inputs/outputs: {port name: shape}; plan: callable enqueuing the kernels on the current
        stream; buffers: {port name: device tensor}."""
        self._inputs = dict(inputs)
        self._outputs = dict(outputs)
        self._plan = plan
        self._buf = buffers
        self._shares: list[tuple[str, str]] = []    # copied after each execute
        self._aliases: list[tuple[str, str]] = []   # written in place
        self._alias_hooks = None                    # (in-place check, re-lowering) from the compiler
        self._executed = False
        self._graph = None
        self.stream = torch.cuda.Stream()

    # -- ports --
    def _port(self, name, table, kind):
        if name not in table:
            raise KeyError(f"unknown {kind} port: {name!r}")
        return self._buf[name]

    def set_input(self, name: str, arr) -> None:
        buf = self._port(name, self._inputs, "input")
        a = np.asarray(arr)
        if tuple(a.shape) != tuple(self._inputs[name]):
            raise ValueError(f"input {name!r}: expected {self._inputs[name]}, got {tuple(a.shape)}")
        with torch.cuda.stream(self.stream):
            buf.copy_(torch.from_numpy(np.ascontiguousarray(a.astype(np.float16))), non_blocking=False)

    def read_output(self, name: str) -> np.ndarray:
        buf = self._port(name, self._outputs, "output")
        self.stream.synchronize()
        return buf.cpu().numpy().astype(np.float16).reshape(self._outputs[name]).copy()

    def input_view(self, name: str) -> torch.Tensor:
        return self._port(name, self._inputs, "input")

    def output_view(self, name: str) -> torch.Tensor:
        return self._port(name, self._outputs, "output")

    def share_buffer(self, src_op_idx: int, src_out_port: str, dst_op_idx: int, dst_in_port: str) -> None:
        """Keep `src_out_port` resident as `dst_in_port` across executes (aneforge/_runtime.py:185-195)."""
        if self._executed:
            raise RuntimeError("share_buffer must be called before the first execute")
        src = self._port(src_out_port, self._outputs, "output")
        dst = self._port(dst_in_port, self._inputs, "input")
        if tuple(src.shape) != tuple(dst.shape):
            raise RuntimeError(f"share_buffer({src_out_port}->{dst_in_port}): shapes {tuple(src.shape)} vs {tuple(dst.shape)}")
        if any(d == dst_in_port for _, d in self._shares + self._aliases):
            raise RuntimeError(f"share_buffer: input {dst_in_port!r} is already shared")
        if self._alias_hooks is not None and self._alias_hooks[0](src_out_port, dst_in_port):
            self._aliases.append((src_out_port, dst_in_port))
            self._plan, self._buf = self._alias_hooks[1](self._aliases)
        else:
            self._shares.append((src_out_port, dst_in_port))

    def shared_in_place(self, out_port: str) -> bool:
        """True when share_buffer aliased this output onto its input (no per-execute copy)."""
        return any(o == out_port for o, _ in self._aliases)

    # -- execution --
    def _enqueue(self):
        from . import _kernels as K
        self._plan()
        for s, d in self._shares:               # device-to-device, as a capturable copy kernel
            n = self._buf[s].numel()
            K.copy_strided(self._buf[s], [1], [n], dst=self._buf[d], dst_strides=[1])

    def execute(self) -> None:
        self._executed = True
        with torch.cuda.stream(self.stream):
            if self._graph is None:
                self._graph = _capture(self.stream, self._enqueue)
            if self._graph is not None:
                _hip.call("afx_graph_launch", self._graph, self.stream.cuda_stream)
            else:
                self._enqueue()
        self.stream.synchronize()

    def eval(self, inputs: dict) -> dict:
        for name, arr in inputs.items():
            self.set_input(name, arr)
        self.execute()
        return {name: self.read_output(name) for name in self._outputs}

    def release(self) -> None:
        if self._graph is not None:
            _hip.call("afx_graph_destroy", self._graph)
            self._graph = None
        self._buf = {}

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.release()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


def _capture(stream, fn):
    """Capture fn's launches into a HIP graph on `stream`; None if capture is not possible."""
    ex = ctypes.c_void_p()
    try:
        _hip.call("afx_graph_begin", stream.cuda_stream)
    except RuntimeError:
        return None
    ok = True
    try:
        fn()
    except Exception:
        ok = False
        raise
    finally:
        try:
            _hip.call("afx_graph_end", stream.cuda_stream, ctypes.byref(ex))
        except RuntimeError:
            ok = False
    return ex if ok and ex.value else None
