"""cq35_step_static (the decode step that allocates nothing: its scratch is a
static device array) against cq35_step on the same state: greedy token,
BF16 logits and the updated state bit for bit, on two calls in a row, the
second with a smaller state (capacity) than the first."""
import ctypes

import numpy as np
import pytest

import cq35
import cq35.config as cc
from cq35 import _lib

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


class DeviceBuffer:
    """Caller-owned device memory for the state (allocated by the test, not by
    the entry point under test)."""

    def __init__(self, nbytes: int):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.ptr = ctypes.c_void_p()
        self.nbytes = nbytes
        assert self.hip.hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(nbytes)) == 0

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes == self.nbytes
        assert self.hip.hipMemcpy(self.ptr, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) == 0

    def download(self, dtype) -> np.ndarray:
        out = np.empty(self.nbytes // np.dtype(dtype).itemsize, dtype=dtype)
        assert self.hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, ctypes.c_size_t(self.nbytes), 2) == 0
        return out

    def free(self):
        if self.ptr:
            self.hip.hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()


def static_step(model, buf, capacity, token, start):
    lib = _lib.load()
    nxt = ctypes.c_uint64()
    logits = np.empty(model.vocabulary_size, dtype=np.uint16)
    _lib.check(lib.cq35_step_static(model._h, buf.ptr, capacity, token, start, None,
                                    ctypes.byref(nxt), logits.ctypes.data))
    return int(nxt.value), logits


_models = {}


def model_of(name):
    if name not in _models:
        _models[name] = cq35.Model.synthetic(cc.preset(name), seed=7)
    return _models[name]


@pytest.mark.parametrize("name", ["tiny-moe", "mini-moe", "tiny", "qwen36-35b-a3b"])
def test_static_step_matches_session_step(name):
    cfg = cc.preset(name)
    model = model_of(name)
    rng = np.random.default_rng(3)
    for capacity, plen in [(96, 40), (24, 5)]:  # the second call is smaller
        say("static step", name, "capacity", capacity, "position", plen)
        prompt = rng.integers(0, cfg["vocab"], plen).tolist()
        s = model.session(capacity)
        for t in prompt:  # one token per call: the same decode kernels on both sides
            tok = s.append_next_token([t])
        before = s.export_state(0)
        buf = DeviceBuffer(before.nbytes)
        buf.upload(before)
        got_tok, got_logits = static_step(model, buf, capacity, tok, plen)
        ref_logits, ref_tok = s.step_raw([tok])
        assert got_tok == ref_tok, (name, capacity)
        assert np.array_equal(got_logits, ref_logits), (name, capacity)
        assert np.array_equal(buf.download(np.uint16), s.export_state(0)), (name, capacity)
        buf.free()


def test_static_steps_from_two_threads_serialise():
    """Two threads step two different caller-owned states through
    cq35_step_static at the same time (ctypes releases the GIL during the
    call, so the calls overlap on the host): each call holds the device's
    lock until its stream has drained, so each thread's tokens, logits and
    final state equal the same steps taken by cq35_step on a session."""
    import threading
    name, capacity, steps = "mini-moe", 64, 8
    cfg = cc.preset(name)
    model = model_of(name)
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, cfg["vocab"], 6).tolist() for _ in range(2)]
    starts, bufs, firsts, refs = [], [], [], []
    for p in prompts:
        s = model.session(capacity)
        for t in p:
            tok = s.append_next_token([t])
        buf = DeviceBuffer(s.state_bytes(0))
        buf.upload(s.export_state(0))
        bufs.append(buf)
        firsts.append(tok)
        starts.append(len(p))
        calls, t = [], tok
        for _ in range(steps):
            lg, t = s.step_raw([t])
            calls.append((t, lg))
        refs.append((calls, s.export_state(0)))
    got = [[] for _ in prompts]
    errors = []
    barrier = threading.Barrier(2)

    def worker(i):
        try:
            barrier.wait()
            t = firsts[i]
            for k in range(steps):
                t, lg = static_step(model, bufs[i], capacity, t, starts[i] + k)
                got[i].append((t, lg))
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for i, (calls, state) in enumerate(refs):
        say("static step thread", i)
        for k, ((gt, gl), (rt, rl)) in enumerate(zip(got[i], calls)):
            assert gt == rt and np.array_equal(gl, rl), (i, k)
        assert np.array_equal(bufs[i].download(np.uint16), state), i
        bufs[i].free()


def test_static_step_rejects_bad_arguments():
    cfg = cc.preset("qwen36-35b-a3b")
    model = model_of("qwen36-35b-a3b")
    lib = _lib.load()
    nxt = ctypes.c_uint64()
    buf = DeviceBuffer(model.session(8).state_bytes(0))
    # position outside the capacity, token outside the vocabulary: rejected before any work
    assert lib.cq35_step_static(model._h, buf.ptr, 8, 1, 8, None, ctypes.byref(nxt), None) == -2
    assert lib.cq35_step_static(model._h, buf.ptr, 8, cfg["vocab"], 0, None, ctypes.byref(nxt), None) == -2
    # a capacity whose attention partials do not fit the static scratch
    # (16 query heads x ~3 floats per position); nothing is launched
    assert lib.cq35_step_static(model._h, buf.ptr, 262144, 1, 0, None, ctypes.byref(nxt), None) == -2
    assert b"static maximum" in lib.cq35_last_error()
    buf.free()
    _models.clear()
