"""Stream-ordered host calls (vbm_host_call_*): the HIP side of the reference's GGML_OP_CUSTOM
host-call node (llama-b11669-hybrid-experts.patch:82-101, :800-1054). CPU: descriptor layout and
argument checks. GPU: both modes, join nodes, miss-only bookkeeping posts, graph replays and the
bounded mailbox wait (forced to expire from the host with a tiny poll limit)."""
import ctypes as C
import time

import numpy as np
import pytest


def test_descriptor_layout_matches_ggml_host_call(vb):
    # ggml_host_call: u64 magic, fn, ctx, src_host[GGML_MAX_SRC = 10], dst_host, backend_state,
    # call, int32 miss_src (patch :88-100), natural alignment on LP64
    H = vb.HostCall
    assert H.magic.offset == 0 and H.fn.offset == 8 and H.ctx.offset == 16 and H.src_host.offset == 24
    assert H.dst_host.offset == 24 + 8 * 10 and H.backend_state.offset == 112 and H.call.offset == 120
    assert H.miss_src.offset == 128 and C.sizeof(H) == 136
    assert vb.HOST_CALL_MAGIC.to_bytes(8, "big") == b"VBHCALL1" and vb.HOST_JOIN_MAGIC.to_bytes(8, "big") == b"VBHJOIN1"
    text = vb.HEADER.read_text()
    assert "#define VBM_HOST_MAX_SRC 10" in text and "0x56424843414c4c31ULL" in text


def test_enqueue_rejects_bad_descriptors_before_device_work(vb):
    call = vb.HostCall()
    dst = C.c_void_p(1)
    with pytest.raises(vb.VbmError, match="descriptor"):
        vb.call("vbm_host_call_enqueue", C.byref(call), None, None, 0, dst, 4, None, 0, 0, None)
    call.magic = vb.HOST_CALL_MAGIC
    with pytest.raises(vb.VbmError, match="needs fn"):
        vb.call("vbm_host_call_enqueue", C.byref(call), None, None, 0, dst, 4, None, 0, 0, None)
    call.fn = vb.HOST_FN(lambda ctx: None)
    call.dst_host = 1
    srcs = (C.c_void_p * 1)(8)
    sizes = (C.c_size_t * 1)(4)
    with pytest.raises(vb.VbmError, match="host buffer"):
        vb.call("vbm_host_call_enqueue", C.byref(call), srcs, sizes, 1, dst, 4, None, 0, 0, None)
    with pytest.raises(vb.VbmError, match="inputs"):
        vb.call("vbm_host_call_enqueue", C.byref(call), srcs, sizes, 11, dst, 4, None, 0, 0, None)
    with pytest.raises(vb.VbmError, match="mode"):
        vb.call("vbm_host_call_enqueue", C.byref(call), None, None, 0, dst, 4, None, 0, 7, None)
    with pytest.raises(vb.VbmError, match="mailbox"):
        vb.call("vbm_host_call_enqueue", C.byref(call), None, None, 0, dst, 4, C.c_void_p(8), 2, 0, None)
    with pytest.raises(vb.VbmError, match="never enqueued"):
        vb.call("vbm_host_join", C.byref(call), dst, dst, dst, 1, None)


class Pinned:
    def __init__(self, vb, n):
        self.vb, self.n = vb, n
        p = C.c_void_p()
        vb.call("vbm_host_alloc", C.byref(p), 4 * n)
        self.ptr = p.value
        self.arr = np.ctypeslib.as_array((C.c_float * n).from_address(self.ptr))

    def free(self):
        self.vb.call("vbm_host_free", self.ptr)


class AxpyCall:
    """dst_host = 2 * src0 + src1 (fp32, n), counting its runs."""

    def __init__(self, vb, n):
        self.vb, self.n = vb, n
        self.src = [Pinned(vb, n), Pinned(vb, n)]
        self.dst = Pinned(vb, n)
        self.runs = 0
        self.delay = 0.0

        def fn(ctx):
            if self.delay:
                time.sleep(self.delay)
            self.dst.arr[:] = 2.0 * self.src[0].arr + self.src[1].arr
            self.runs += 1

        self.fn = vb.HOST_FN(fn)
        self.call = vb.HostCall()
        self.call.magic = vb.HOST_CALL_MAGIC
        self.call.fn = self.fn
        self.call.src_host[0], self.call.src_host[1] = self.src[0].ptr, self.src[1].ptr
        self.call.dst_host = self.dst.ptr

    def enqueue(self, a, b, out, mode, miss=None, n_miss=0, stream=None, wait=False):
        """wait: make `stream` wait for the call (the call runs on a side stream; without a join or
        a wait, synchronizing `stream` does not cover it)."""
        vb = self.vb
        srcs = (C.c_void_p * 2)(a.ptr, b.ptr)
        sizes = (C.c_size_t * 2)(4 * self.n, 4 * self.n)
        vb.call("vbm_host_call_enqueue", C.byref(self.call), srcs, sizes, 2, out.ptr, 4 * self.n,
                None if miss is None else miss.ptr, n_miss, mode, stream)
        if wait:
            vb.call("vbm_host_call_wait", C.byref(self.call), stream)

    def release(self):
        self.vb.call("vbm_host_call_release", C.byref(self.call))
        for p in self.src + [self.dst]:
            p.free()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_host_call_and_join(gpu, mode):
    vb = gpu
    n = 4096
    rng = np.random.default_rng(mode)
    a_h, b_h, c_h = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    a, b, c = (vb.DeviceBuffer.from_array(v) for v in (a_h, b_h, c_h))
    mid, out = vb.DeviceBuffer(4 * n), vb.DeviceBuffer(4 * n)
    call = AxpyCall(vb, n)
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    call.enqueue(a, b, mid, mode, stream=stream.value)
    vb.call("vbm_host_join", C.byref(call.call), mid.ptr, c.ptr, out.ptr, n, stream.value)
    vb.call("vbm_stream_synchronize", stream.value)
    assert np.array_equal(mid.download(np.float32, n), 2 * a_h + b_h)
    assert np.array_equal(out.download(np.float32, n), (2 * a_h + b_h) + c_h)
    assert call.runs == 1
    call.release()
    vb.call("vbm_stream_destroy", stream.value)


@pytest.mark.gpu
def test_mailbox_miss_only_posts_are_not_waited_for(gpu):
    vb = gpu
    n = 1024
    a_h = np.arange(n, dtype=np.float32)
    a, b = vb.DeviceBuffer.from_array(a_h), vb.DeviceBuffer.from_array(np.ones(n, np.float32))
    out = vb.DeviceBuffer.from_array(np.full(n, 7.0, np.float32))
    call = AxpyCall(vb, n)
    hits = vb.DeviceBuffer.from_array(np.array([1, 1, 1, 1], np.int32))      # no miss: bookkeeping only
    call.enqueue(a, b, out, vb.HOST_CALL_MAILBOX, miss=hits, n_miss=4, wait=True)
    vb.call("vbm_stream_synchronize", None)
    assert not out.download(np.float32, n).any()
    vb.call("vbm_host_mailbox_drain", 0, 10.0)
    assert call.runs == 1                                                    # fn still ran
    misses = vb.DeviceBuffer.from_array(np.array([1, 0, 1], np.int32))      # one miss: waited
    call.enqueue(a, b, out, vb.HOST_CALL_MAILBOX, miss=misses, n_miss=3, wait=True)
    vb.call("vbm_stream_synchronize", None)
    assert np.array_equal(out.download(np.float32, n), 2 * a_h + 1) and call.runs == 2
    posted, done, timeouts = C.c_uint64(), C.c_uint64(), C.c_uint32()
    vb.call("vbm_host_mailbox_stats", 0, C.byref(posted), C.byref(done), C.byref(timeouts))
    assert done.value == posted.value and posted.value >= 2
    call.release()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_host_call_graph_replays(gpu, mode):
    vb = gpu
    n = 2048
    a, b, c = vb.DeviceBuffer(4 * n), vb.DeviceBuffer(4 * n), vb.DeviceBuffer(4 * n)
    mid, out = vb.DeviceBuffer(4 * n), vb.DeviceBuffer(4 * n)
    call = AxpyCall(vb, n)
    vb.call("vbm_host_call_prepare", C.byref(call.call), mode)
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    s = stream.value
    vb.call("vbm_graph_begin_capture", s)
    call.enqueue(a, b, mid, mode, stream=s)
    vb.call("vbm_host_join", C.byref(call.call), mid.ptr, c.ptr, out.ptr, n, s)
    graph = C.c_void_p()
    vb.call("vbm_graph_end_capture", s, C.byref(graph))
    rng = np.random.default_rng(10 + mode)
    for rep in range(4):
        vals = [rng.standard_normal(n).astype(np.float32) for _ in range(3)]
        for buf, v in zip((a, b, c), vals):
            buf.upload(v)
        vb.call("vbm_device_synchronize")
        vb.call("vbm_graph_launch", graph.value, s)
        vb.call("vbm_stream_synchronize", s)
        assert np.array_equal(out.download(np.float32, n), (2 * vals[0] + vals[1]) + vals[2]), rep
    assert call.runs == 4
    vb.call("vbm_graph_destroy", graph.value)
    call.release()
    vb.call("vbm_stream_destroy", s)


@pytest.mark.gpu
def test_mailbox_wait_is_bounded(gpu):
    vb = gpu
    n = 256
    a, b = vb.DeviceBuffer.from_array(np.ones(n, np.float32)), vb.DeviceBuffer.from_array(np.ones(n, np.float32))
    out = vb.DeviceBuffer.from_array(np.full(n, 5.0, np.float32))
    call = AxpyCall(vb, n)
    call.delay = 0.2                        # far longer than 50 polls of ~1 us
    before = C.c_uint32()
    vb.call("vbm_host_mailbox_stats", 0, None, None, C.byref(before))
    vb.call("vbm_host_mailbox_set_spin_limit", 50)
    try:
        call.enqueue(a, b, out, vb.HOST_CALL_MAILBOX, wait=True)
        vb.call("vbm_stream_synchronize", None)
    finally:
        vb.call("vbm_host_mailbox_set_spin_limit", 1 << 21)
    after = C.c_uint32()
    vb.call("vbm_host_mailbox_stats", 0, None, None, C.byref(after))
    assert after.value == before.value + 1
    assert not out.download(np.float32, n).any()          # an expired wait zero-fills the output
    vb.call("vbm_host_mailbox_drain", 0, 10.0)
    assert call.runs == 1
    call.release()


@pytest.mark.gpu
def test_mailbox_reenqueue_and_release_wait_for_an_unwaited_post(gpu):
    """A bookkeeping-only post (no miss, not waited for) whose fn is still sleeping when the same
    descriptor is enqueued again with new inputs: fn must read the inputs of its own post (the new
    input copies wait until the worker has handled the previous post), and release must not return
    while fn is still queued or running."""
    vb = gpu
    n = 512
    seen = []
    call = AxpyCall(vb, n)
    inner = call.fn

    def observing(ctx):
        import time as _t
        _t.sleep(0.05)
        seen.append(float(call.src[0].arr[0]))
        inner(ctx)
    call.fn = vb.HOST_FN(observing)
    call.call.fn = call.fn
    ones = vb.DeviceBuffer.from_array(np.ones(n, np.float32))
    a1 = vb.DeviceBuffer.from_array(np.full(n, 1.0, np.float32))
    a2 = vb.DeviceBuffer.from_array(np.full(n, 2.0, np.float32))
    out = vb.DeviceBuffer(4 * n)
    hits = vb.DeviceBuffer.from_array(np.array([1, 1], np.int32))          # no miss: not waited for
    call.enqueue(a1, ones, out, vb.HOST_CALL_MAILBOX, miss=hits, n_miss=2, wait=True)
    call.enqueue(a2, ones, out, vb.HOST_CALL_MAILBOX, wait=True)           # waited, new inputs
    vb.call("vbm_stream_synchronize", None)
    assert np.array_equal(out.download(np.float32, n), np.full(n, 5.0, np.float32))
    vb.call("vbm_host_mailbox_drain", 0, 10.0)
    assert seen == [1.0, 2.0], seen
    # release right after an unwaited post: returns only once its fn has run
    call.enqueue(a1, ones, out, vb.HOST_CALL_MAILBOX, miss=hits, n_miss=2, wait=True)
    vb.call("vbm_stream_synchronize", None)
    vb.call("vbm_host_call_release", C.byref(call.call))
    assert seen == [1.0, 2.0, 1.0], seen
    for p in call.src + [call.dst]:
        p.free()
