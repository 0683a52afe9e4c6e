"""Whole-model decode driver (model.rs TextForCausalLM + the greedy loop of main.rs:100-132).

The model, its caches and the captured decode-step graph live in libq35.so; this class only
owns the handle.
"""
import atexit
import ctypes
import weakref

import numpy as np

from . import _lib as L

_live = weakref.WeakSet()


@atexit.register
def _close_all():
    """Destroy every model still open while the interpreter and the HIP runtime are fully up
    (atexit handlers run before module teardown and long before the C runtime's exit
    handlers), so no device memory is freed from a finaliser during shutdown."""
    for m in list(_live):
        m.close()


class TextForCausalLM:
    def __init__(self, dims=None, seed=0, tmax=2048):
        self.dims = dims if dims is not None else L.dims_2b()
        self.seed, self.tmax = seed, tmax
        h = ctypes.c_void_p()
        L.check(L.lib().q35_model_create_synthetic(ctypes.byref(self.dims), seed, tmax, ctypes.byref(h)))
        self.h = h
        _live.add(self)

    @classmethod
    def from_safetensors(cls, path, dims=None, tmax=2048):
        """The decoder with the weights of a Hugging Face safetensors checkpoint (main.rs:160-222
        ingestion: key remap, [out][in] -> [in][out], f32, Q8F per block of 64)."""
        self = cls.__new__(cls)
        self.dims = dims if dims is not None else L.dims_2b()
        self.seed, self.tmax = None, tmax
        h = ctypes.c_void_p()
        L.check(L.lib().q35_model_create_from_safetensors(ctypes.byref(self.dims), str(path).encode(), tmax,
                                                          ctypes.byref(h)))
        self.h = h
        _live.add(self)
        return self

    def close(self):
        if self.h:
            L.lib().q35_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        L.check(L.lib().q35_model_reset(self.h, None))

    def set_token(self, token):
        L.check(L.lib().q35_model_set_token(self.h, int(token), None))

    MODES = {"stream": L.Q35_LAUNCH_STREAM, "graph": L.Q35_LAUNCH_GRAPH, "persistent": L.Q35_LAUNCH_PERSISTENT}

    def _mode(self, mode, use_graph):
        """Launch mode: `mode` ("stream" | "graph" | "persistent"), else the legacy use_graph
        flag (True -> graph, False -> stream), else the persistent kernel."""
        if mode is not None:
            return self.MODES[mode] if isinstance(mode, str) else int(mode)
        if use_graph is not None:
            return L.Q35_LAUNCH_GRAPH if use_graph else L.Q35_LAUNCH_STREAM
        return L.Q35_LAUNCH_PERSISTENT

    def persistent_grid(self):
        """Blocks of the persistent step kernel; raises Q35Error if it cannot run here."""
        g = ctypes.c_int32(0)
        L.check(L.lib().q35_model_persistent_info(self.h, ctypes.byref(g)))
        return g.value

    def step(self, use_graph=None, mode=None, stream=None):
        L.check(L.lib().q35_model_step(self.h, self._mode(mode, use_graph), stream))

    def decode(self, n_steps, mode=None, stream=None):
        """n_steps decode steps, asynchronous on `stream` (a hipStream_t value; None = the model's
        own stream); one launch in persistent mode."""
        L.check(L.lib().q35_model_decode(self.h, int(n_steps), self._mode(mode, None), stream))

    def check(self, stream=None):
        """Synchronise and raise if a persistent launch failed."""
        L.check(L.lib().q35_model_check(self.h, stream))

    def decode_stream(self, max_steps, stop_ids=(), stream=None, wait_s=30.0):
        """Up to max_steps decode steps as one persistent launch, yielding each token (the argmax
        after each step) as the running kernel stores it into the model's pinned host token stream
        (q35_model_decode_stream): the host sees every token as it is made, with no per-step
        synchronisation.  The same tokens as decode() leaves in hist.  With stop ids the launch
        ends before a step whose input token is one of them: the stop id is the last token
        yielded (none, if the current token already is one).  The launch is checked and the
        position updated (q35_model_stream_end) when the generator finishes or is closed; a token
        that does not arrive within wait_s seconds raises."""
        import time
        stops = [int(v) for v in stop_ids]
        s = np.ascontiguousarray(np.asarray(stops, dtype=np.int32))
        if stops:
            self.check(stream)
            if int(self.tensor("token", np.int32)[0]) in stops:
                return
        p0 = self.position()
        L.check(L.lib().q35_model_decode_stream(self.h, int(max_steps), s.ctypes.data if s.size else None, s.size,
                                                stream))
        try:
            if max_steps > 0:
                slots = (ctypes.c_int32 * (p0 + int(max_steps))).from_address(L.lib().q35_model_token_stream(self.h))
            for q in range(p0, p0 + int(max_steps)):
                t0 = time.monotonic()
                while slots[q] < 0:
                    if time.monotonic() - t0 > wait_s:
                        raise RuntimeError(f"decode_stream: no token for position {q} after {wait_s} s")
                tok = int(slots[q])
                yield tok
                if tok in stops:
                    break
        finally:
            n = ctypes.c_int32(0)
            L.check(L.lib().q35_model_stream_end(self.h, ctypes.byref(n), stream))

    def generate(self, prompt, n_new, use_graph=None, readback_each=False, mode=None, stream=None, prefill=False):
        """Returns (tokens[n_new+1], decode_seconds): the argmax after the last prompt token,
        then the argmax after each of n_new decode steps.  prefill=True feeds the prompt through
        the prompt path (GEMMs, chunked delta rule) instead of one decode step per token."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = np.zeros(n_new + 1, np.int32)
        secs = ctypes.c_double(0.0)
        m = self._mode(mode, use_graph) | (L.Q35_PREFILL_GEMM if prefill else 0)
        L.check(L.lib().q35_model_generate(self.h, p.ctypes.data, p.size, n_new, out.ctypes.data, m,
                                           1 if readback_each else 0, ctypes.byref(secs), stream))
        return out, secs.value

    def generate_until(self, prompt, max_new, stop_ids=(), mode=None, stream=None, prefill=False):
        """The chat loop's generation (main.rs:100-132): returns (produced, last, decode_seconds),
        `produced` the ids forwarded after the prompt (at most max_new) and `last` the id that
        ended the loop (a stop id, or the argmax after the last produced id)."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        s = np.ascontiguousarray(np.asarray(list(stop_ids), dtype=np.int32))
        out = np.zeros(max_new + 1, np.int32)
        n = ctypes.c_int32(0)
        secs = ctypes.c_double(0.0)
        m = self._mode(mode, None) | (L.Q35_PREFILL_GEMM if prefill else 0)
        L.check(L.lib().q35_model_generate_until(self.h, p.ctypes.data, p.size, int(max_new),
                                                 s.ctypes.data if s.size else None, s.size, out.ctypes.data,
                                                 ctypes.byref(n), m, ctypes.byref(secs), stream))
        return out[:n.value].copy(), int(out[n.value]), secs.value

    def decode_until(self, max_new, stop_ids=(), mode=None, stream=None):
        """Greedy steps from the current token slot until a stop id or max_new steps: returns
        (produced, last, decode_seconds) as generate_until does."""
        s = np.ascontiguousarray(np.asarray(list(stop_ids), dtype=np.int32))
        out = np.zeros(max_new + 1, np.int32)
        n = ctypes.c_int32(0)
        secs = ctypes.c_double(0.0)
        L.check(L.lib().q35_model_decode_until(self.h, int(max_new), s.ctypes.data if s.size else None, s.size,
                                               out.ctypes.data, ctypes.byref(n), self._mode(mode, None),
                                               ctypes.byref(secs), stream))
        return out[:n.value].copy(), int(out[n.value]), secs.value

    def prefill(self, prompt, stream=None):
        """Feeds the prompt as one forward at seq_len = len(prompt) (the prompt path); the argmax
        after its last token is left in the token slot.  Asynchronous after the upload."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        L.check(L.lib().q35_model_prefill(self.h, p.ctypes.data, p.size, stream))

    def current_token(self, stream=None):
        """The token slot: the input of the next decode step (the argmax after the last one, or
        after the prompt).  Synchronises."""
        self.check(stream)
        return int(self.tensor("token", np.int32)[0])

    def position(self):
        v = ctypes.c_int32(0)
        L.check(L.lib().q35_model_position(self.h, ctypes.byref(v)))
        return v.value

    def tensor_ptr(self, name):
        ptr = ctypes.c_void_p()
        nbytes = ctypes.c_size_t()
        L.check(L.lib().q35_model_tensor(self.h, name.encode(), ctypes.byref(ptr), ctypes.byref(nbytes)))
        return ptr.value, nbytes.value

    def tensor(self, name, dtype, shape=None):
        """Copy of a model tensor as a numpy array (synchronises the device)."""
        import torch
        ptr, nbytes = self.tensor_ptr(name)
        torch.cuda.synchronize()
        n = nbytes // np.dtype(dtype).itemsize
        out = np.empty(n, dtype)
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        rc = hip.hipMemcpy(out.ctypes.data, ctypes.c_void_p(ptr), nbytes, 2)  # hipMemcpyDeviceToHost
        if rc != 0:
            raise RuntimeError(f"hipMemcpy failed: {rc}")
        return out.reshape(shape) if shape is not None else out

    def set_tensor(self, name, values):
        """Overwrite a model tensor with host values of the same byte size (synchronises)."""
        import torch
        ptr, nbytes = self.tensor_ptr(name)
        v = np.ascontiguousarray(values)
        if v.nbytes > nbytes:
            raise ValueError(f"{name}: {v.nbytes} bytes given, tensor holds {nbytes}")
        torch.cuda.synchronize()
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        rc = hip.hipMemcpy(ctypes.c_void_p(ptr), v.ctypes.data, v.nbytes, 1)  # hipMemcpyHostToDevice
        if rc != 0:
            raise RuntimeError(f"hipMemcpy failed: {rc}")


def synth_model_tensor(dims, seed, name, n):
    """f32 values the model builder draws for tensor `name` (before Q8F quantisation)."""
    out = np.empty(n, np.float32)
    L.check(L.lib().q35_synth_model_tensor(ctypes.byref(dims), seed, name.encode(), out.ctypes.data, n))
    return out


class BatchDecoder:
    """B sequences decoded together with the weights of `model` (a TextForCausalLM), each with
    its own caches, position and history (q35_batch_*)."""

    def __init__(self, model, B, tmax=None):
        self.model, self.B = model, int(B)
        self.tmax = int(tmax if tmax is not None else model.tmax)
        h = ctypes.c_void_p()
        L.check(L.lib().q35_batch_create(model.h, self.B, self.tmax, ctypes.byref(h)))
        self.h = h
        _live.add(self)

    def close(self):
        if self.h:
            L.lib().q35_batch_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        L.check(L.lib().q35_batch_reset(self.h, None))

    def step(self, mode="graph", stream=None):
        L.check(L.lib().q35_batch_step(self.h, TextForCausalLM.MODES[mode], stream))

    def decode(self, n_steps, mode="graph", stream=None):
        L.check(L.lib().q35_batch_decode(self.h, int(n_steps), TextForCausalLM.MODES[mode], stream))

    def generate(self, prompts, n_new, mode="graph", prefill=False, stream=None):
        """prompts: B id sequences (any lengths) -> (tokens [B][n_new + 1], decode_seconds)."""
        assert len(prompts) == self.B
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompts]))
        lens = np.ascontiguousarray(np.array([len(p) for p in prompts], np.int32))
        out = np.zeros((self.B, n_new + 1), np.int32)
        secs = ctypes.c_double(0.0)
        m = TextForCausalLM.MODES[mode] | (L.Q35_PREFILL_GEMM if prefill else 0)
        L.check(L.lib().q35_batch_generate(self.h, flat.ctypes.data, lens.ctypes.data, int(n_new), out.ctypes.data, m,
                                           ctypes.byref(secs), stream))
        return out, secs.value

    def positions(self):
        out = np.zeros(self.B, np.int32)
        L.check(L.lib().q35_batch_position(self.h, out.ctypes.data))
        return out

    def tensor(self, name, dtype):
        import torch
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        L.check(L.lib().q35_batch_tensor(self.h, name.encode(), ctypes.byref(ptr), ctypes.byref(nbytes)))
        torch.cuda.synchronize()
        out = np.empty(nbytes.value // np.dtype(dtype).itemsize, dtype)
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        if hip.hipMemcpy(out.ctypes.data, ptr, nbytes.value, 2) != 0:
            raise RuntimeError("hipMemcpy failed")
        return out


def safetensors_tensor(path, dims, name, n):
    """f32 values the safetensors loader takes for decoder tensor `name` (Linear weights as
    [in][out]), before quantisation; host only."""
    out = np.empty(n, np.float32)
    L.check(L.lib().q35_safetensors_tensor(str(path).encode(), ctypes.byref(dims), name.encode(), out.ctypes.data, n))
    return out


def quantize_q8f(w):
    """Q8F quantiser of the library (blocks of 64 along the last axis)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // 64), np.float32)
    L.check(L.lib().q35_quantize_q8f(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data))
    return q, s


def synth_normal(seed, stream, n, sigma=1.0, offset=0):
    out = np.empty(n, np.float32)
    L.check(L.lib().q35_synth_normal(seed, stream, offset, n, sigma, out.ctypes.data))
    return out


def synth_uniform(seed, stream, n, lo, hi, offset=0):
    out = np.empty(n, np.float32)
    L.check(L.lib().q35_synth_uniform(seed, stream, offset, n, lo, hi, out.ctypes.data))
    return out
