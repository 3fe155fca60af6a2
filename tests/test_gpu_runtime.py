"""GPU behaviour of the runtime boundary (marked `gpu`): handle cache, buffer
pool growth, handle lifetime, typed errors on a live device, the completion
timeout, concurrency, event timing and the autotuner.  Behaviour spec:
crates/axc-runtime/tests (handle reuse, pow2 growth, error paths,
kernel_handle_outlives_context.rs:24, amortisation) of the reference."""
from __future__ import annotations

import struct
import sys
import threading

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _plan(axc, n=3, pc=4, wg=64):
    acc = [axc.axh.ACCESS_READ_ONLY] * (n - 1) + [axc.axh.ACCESS_READ_WRITE]
    return axc.BindingPlan(acc, pc, (wg, 1, 1))


def _q4km_handle(ctx, axc):
    return ctx.prepare_kernel(axc.builtin_code_object(), _plan(axc), 4, "q4km_dequant_matvec")


def test_prepare_twice_returns_cached_handle(ctx, axc):
    h1 = _q4km_handle(ctx, axc)
    h2 = _q4km_handle(ctx, axc)
    assert h1.raw == h2.raw and h1.cache_key == h2.cache_key
    h1.release()
    # still alive through h2
    q, x = O.generate_q4km_test_data(4, 0xDEADBEEF)
    out = ctx.dispatch_handle(h2, (1, 1, 1), [q.tobytes(), x.tobytes(), b""], [0, 0, 4],
                              struct.pack("<I", 4))
    assert O.reference_rel_err(struct.unpack("<f", out[2])[0], O.q4k_dot(q, x, 4)) < 1e-3
    h2.release()
    h3 = _q4km_handle(ctx, axc)  # prepared again after the last release
    assert h3.raw
    h3.release()


def test_buffer_pool_grows_to_pow2_and_never_shrinks(ctx, axc):
    h = _q4km_handle(ctx, axc)
    for n in (1, 2, 1):
        q, x = O.generate_q4km_test_data(n, 7)
        ctx.dispatch_handle(h, (1, 1, 1), [q.tobytes(), x.tobytes(), b""], [0, 0, 4],
                            struct.pack("<I", n))
    # n=2 sized the pools: q 288 -> 512, x 2048 -> 2048, y max(4,4) -> 4
    assert (h.pool_bytes(0), h.pool_bytes(1), h.pool_bytes(2)) == (512, 2048, 4)
    h.release()


def test_handle_outlives_context(axc):
    """AT-827: drop the context first, then the handle; no use after free."""
    c = axc.HipContext.new()
    h = _q4km_handle(c, axc)
    q, x = O.generate_q4km_test_data(2, 1)
    c.dispatch_handle(h, (1, 1, 1), [q.tobytes(), x.tobytes(), b""], [0, 0, 4],
                      struct.pack("<I", 2))
    c.close()
    assert h.pool_bytes(0) == 512  # device state still valid through the handle
    h.release()


def test_dispatch_error_paths_on_device(ctx, axc):
    h = _q4km_handle(ctx, axc)
    with pytest.raises(axc.DispatchError) as e:
        ctx.dispatch_handle(h, (1, 1, 1), [b"", b""], [0, 0, 4], struct.pack("<I", 0))
    assert e.value.variant == "BindingCountMismatch"
    with pytest.raises(axc.DispatchError) as e:
        ctx.dispatch_handle(h, (1, 1, 1), [b"", b"", b""], [0, 0, 4], b"\0" * 8)
    assert e.value.variant == "PushConstantSizeMismatch"
    big = ctx.max_workgroup_count[0] + 1
    if big <= 0xFFFFFFFF:
        with pytest.raises(axc.DispatchError) as e:
            ctx.dispatch_handle(h, (big, 1, 1), [b"", b"", b""], [0, 0, 4], struct.pack("<I", 0))
        assert e.value.variant == "WorkgroupCountExceedsDeviceLimit"
    h.release()


def test_prepare_error_paths_on_device(ctx, axc):
    with pytest.raises(axc.DispatchError) as e:
        ctx.prepare_kernel(b"\x00" * 64, _plan(axc), 4, "q4km_dequant_matvec")
    assert e.value.variant == "ShaderModuleCreationFailed"
    with pytest.raises(axc.DispatchError) as e:
        ctx.prepare_kernel(axc.builtin_code_object(), _plan(axc), 4, "no_such_entry")
    assert e.value.variant == "PipelineCreationFailed"
    with pytest.raises(axc.DispatchError) as e:
        ctx.prepare_kernel(axc.builtin_code_object(), _plan(axc, pc=4), 8, "q4km_dequant_matvec")
    assert e.value.variant == "PipelineLayoutFailed"


def test_fence_timeout_is_reported_and_recoverable(axc):
    """A bounded sleep kernel (~10 ms) against a 1 ms completion timeout."""
    c = axc.HipContext.new_with_options(axc.HipContextOptions(fence_timeout_ms=1))
    h = c.prepare_kernel(axc.builtin_code_object(),
                         axc.BindingPlan([axc.axh.ACCESS_READ_WRITE], 4, (64, 1, 1)), 4, "axh_spin")
    with pytest.raises(axc.DispatchError) as e:
        c.dispatch_handle(h, (1, 1, 1), [b""], [4], struct.pack("<I", 3000))
    assert e.value.variant == "FenceTimeout"
    c.device_synchronize()  # unbounded wait: the bounded kernel ends by itself
    h.release()
    c.close()


def test_spin_kernel_completes_within_default_timeout(ctx, axc):
    h = ctx.prepare_kernel(axc.builtin_code_object(),
                           axc.BindingPlan([axc.axh.ACCESS_READ_WRITE], 4, (64, 1, 1)), 4, "axh_spin")
    out = ctx.dispatch_handle(h, (1, 1, 1), [b""], [4], struct.pack("<I", 10))
    assert struct.unpack("<I", out[0])[0] == 10
    h.release()


@pytest.mark.parametrize("nbytes", [1, 4097, 70 * 1024 * 1024 + 3])
def test_upload_download_round_trip(ctx, nbytes):
    data = np.random.default_rng(nbytes).integers(0, 256, nbytes, dtype=np.uint8)
    b = ctx.alloc(nbytes)
    ctx.upload(b, data)
    assert ctx.download(b, nbytes) == data.tobytes()
    b.close()


def test_concurrent_dispatch_on_two_handles(ctx, axc):
    """Different handles dispatch in parallel; each handle serialises its own."""
    co = axc.builtin_code_object()
    h1 = ctx.prepare_kernel(co, _plan(axc), 4, "q4km_dequant_matvec")
    h2 = ctx.prepare_kernel(co, _plan(axc), 4, "q4_0_dequant_matvec")
    q1, x1 = O.generate_q4km_test_data(8, 3)
    q2 = O.gen_q4_0_weights(4, 16)
    x2 = O.gen_normal_f32(5, 16 * 32)
    ref1, ref2 = O.q4k_dot(q1, x1, 8), O.q4_0_dot(q2, x2, 16)
    errors = []

    def worker(h, q, x, n, ref):
        try:
            for _ in range(30):
                out = ctx.dispatch_handle(h, (1, 1, 1), [q.tobytes(), x.tobytes(), b""], [0, 0, 4],
                                          struct.pack("<I", n))
                if O.reference_rel_err(struct.unpack("<f", out[2])[0], ref) >= 1e-3:
                    errors.append("mismatch")
        except Exception as exc:  # surfaced below
            errors.append(repr(exc))

    ts = [threading.Thread(target=worker, args=(h1, q1, x1, 8, ref1)),
          threading.Thread(target=worker, args=(h2, q2, x2, 16, ref2)),
          threading.Thread(target=worker, args=(h1, q1, x1, 8, ref1))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors[:3]
    h1.release()
    h2.release()


def test_events_time_launches_on_the_context_stream(ctx, axc):
    h = ctx.prepare_kernel(axc.builtin_code_object(),
                           axc.BindingPlan([axc.axh.ACCESS_READ_WRITE], 4, (64, 1, 1)), 4, "axh_spin")
    buf = ctx.alloc(4)
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    ctx.launch(h, (1, 1, 1), [buf], struct.pack("<I", 300))  # ~1 ms of sleeps
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_ms(e1)
    assert 0.1 < ms < 100.0
    assert struct.unpack("<I", ctx.download(buf, 4))[0] == 300
    buf.close()
    h.release()


def test_graph_replays_match_eager_results(ctx, axc):
    """Captured matvec / Q4_0 / matmul launches replayed several times, with
    eager work and synchronisation between replays; every replay is compared
    bit for bit with the eager result.  The Q4_0 launches cover the column,
    one-pass and persistent kernels and the fused gate/up."""
    rows, sb, nb, batch = 300, 16, 128, 24
    q = O.gen_q4k_weights(81, rows * sb)
    x = O.gen_normal_f32(82, sb * 256)
    q0 = O.gen_q4_0_weights(83, rows * nb)
    x0 = O.gen_normal_f32(84, nb * 32)
    xh = O.gen_normal_f32(85, sb * 256 * batch).astype(np.float16)
    # 5 rows of 128 superblocks: the split-K kernel and its workspace counter;
    # the first of them alone: the one-workgroup kernel
    ksb, krows = 128, 5
    qk = O.gen_q4k_weights(86, krows * ksb)
    xk = O.gen_normal_f32(87, ksb * 256)
    rows0b = 1100  # Q4_0 past 1024 rows: the one-pass kernel
    q0b = O.gen_q4_0_weights(88, rows0b * nb)
    bufs = {}
    for name, arr in (("q", q), ("x", x), ("q0", q0), ("x0", x0), ("xh", xh), ("qk", qk),
                      ("xk", xk), ("q0b", q0b)):
        bufs[name] = ctx.alloc(arr.nbytes)
        ctx.upload(bufs[name], arr)
    y1, y2, y3 = ctx.alloc(rows * 4), ctx.alloc(rows * 4), ctx.alloc(rows * batch * 4)
    y4, y5 = ctx.alloc(32), ctx.alloc(16)
    y6, y7, y8 = ctx.alloc(rows0b * 4), ctx.alloc(rows * 4), ctx.alloc(rows * 4)
    outs = ((y1, rows * 4), (y2, rows * 4), (y3, rows * batch * 4), (y4, krows * 4), (y5, 4),
            (y6, rows0b * 4), (y7, rows * 4), (y8, rows * 4))
    persistent = axc.Variant(family=axc.FAMILY_PERSISTENT)
    columns = axc.Variant(family=axc.FAMILY_COLUMNS)
    split_k = axc.Variant(family=axc.FAMILY_SPLIT_K)

    def ops():
        ctx.q4k_matvec(bufs["q"], bufs["x"], y1, rows, sb)
        ctx.q4_0_matvec(bufs["q0"], bufs["x0"], y2, rows, nb, columns)
        ctx.q4k_matmul(bufs["q"], bufs["xh"], y3, rows, sb, batch)
        ctx.q4k_matvec(bufs["qk"], bufs["xk"], y4, krows, ksb, split_k)
        ctx.q4k_matvec(bufs["qk"], bufs["xk"], y5, 1, ksb)
        ctx.q4_0_matvec(bufs["q0b"], bufs["x0"], y6, rows0b, nb)
        ctx.q4_0_gate_up(bufs["q0"], bufs["q0b"], bufs["x0"], y7, rows, nb)
        ctx.q4_0_matvec(bufs["q0"], bufs["x0"], y8, rows, nb, persistent)

    assert axc.q4k_matvec_kernel_name(krows, ksb, split_k).startswith("axh_q4k_matvec_sk_")
    assert axc.q4_0_matvec_kernel_name(rows0b, nb) == "axh_q4_0_matvec_one_i2"
    assert axc.q4k_matvec_kernel_name(1, ksb).startswith("axh_q4k_matvec_wg_")
    ops()  # eager (also prepares every kernel and the workspace before capture)
    ctx.synchronize()
    eager = [ctx.download(b, n) for b, n in outs]
    g = ctx.capture(ops)
    assert g.node_count == 8
    for rep in range(4):
        for b, n in outs:
            ctx.upload(b, np.full(n // 4, np.nan, dtype=np.float32))  # poison between replays
        ctx.q4k_matvec(bufs["q"], bufs["x"], y1, rows, sb)  # eager work between replays
        ctx.q4k_matvec(bufs["qk"], bufs["xk"], y4, krows, ksb, split_k)
        ctx.synchronize()
        g.launch()
        ctx.synchronize()
        got = [ctx.download(b, n) for b, n in outs]
        assert got == eager, f"replay {rep}"
    # The split-K launch is bound to the context stream's workspace: a replay
    # on another stream is refused before any work is queued.  A graph
    # without it replays anywhere.
    other = axc.HipContext.new()
    with pytest.raises(axc.DispatchError) as e:
        g.launch(stream=other.stream)
    assert e.value.variant == "InvalidArgument"
    g.close()
    g2 = ctx.capture(lambda: ctx.q4k_matvec(bufs["q"], bufs["x"], y1, rows, sb))
    ctx.upload(y1, np.full(rows, np.nan, dtype=np.float32))
    g2.launch(stream=other.stream)
    other.synchronize(other.stream)
    assert ctx.download(y1, rows * 4) == eager[0]
    g2.close()
    other.close()
    for b in list(bufs.values()) + [y1, y2, y3, y4, y5, y6, y7, y8]:
        b.close()


def test_staged_upload_after_a_timed_out_upload(axc, ctx):
    """An upload whose copy waits behind a ~10 ms kernel times out (1 ms
    fence); a second upload to another buffer follows at once.  Once the
    device drains, each buffer holds its own bytes: the queued first copy
    still reads the staging memory it was given."""
    c = axc.HipContext.new_with_options(axc.HipContextOptions(fence_timeout_ms=1))
    h = c.prepare_kernel(axc.builtin_code_object(),
                         axc.BindingPlan([axc.axh.ACCESS_READ_WRITE], 4, (64, 1, 1)), 4, "axh_spin")
    flag = c.alloc(4)
    n = 4096
    a, b = c.alloc(n), c.alloc(n)
    da = np.full(n, 0xA5, dtype=np.uint8)
    db = np.full(n, 0x3C, dtype=np.uint8)
    c.launch(h, (1, 1, 1), [flag], struct.pack("<I", 3000))  # bounded: ends by itself
    with pytest.raises(axc.DispatchError) as e:
        c.upload(a, da)
    assert e.value.variant == "FenceTimeout"
    try:
        c.upload(b, db)
    except axc.DispatchError as e2:  # may also wait behind the kernel
        assert e2.variant == "FenceTimeout"
    c.device_synchronize()  # unbounded wait
    assert ctx.download(a, n) == da.tobytes()
    assert ctx.download(b, n) == db.tobytes()
    for buf in (flag, a, b):
        buf.close()
    h.release()
    c.close()


@pytest.mark.parametrize("nbytes", [16, 1 << 20, (1 << 20) + 48, 33030144])
def test_read_floor_reads_every_byte(ctx, axc, nbytes):
    """The bench's launch-floor helper reads exactly the bytes it is given:
    the XOR of its per-wave results equals the XOR of every dword."""
    words = 8 * ctx.cu_count()
    assert words >= 8
    data = np.random.default_rng(nbytes).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    dq, dout = ctx.alloc(nbytes), ctx.alloc(words * 4)
    ctx.upload(dq, data)
    ctx.read_floor(dq, nbytes, dout, words)
    ctx.launch_empty(dout, words)  # writes nothing
    ctx.synchronize()
    got = np.frombuffer(ctx.download(dout, words * 4), dtype=np.uint32)
    assert int(np.bitwise_xor.reduce(got)) == int(np.bitwise_xor.reduce(data))
    with pytest.raises(axc.DispatchError):
        ctx.read_floor(dq, 15, dout, words)  # not a multiple of 16
    with pytest.raises(axc.DispatchError):
        ctx.read_floor(dq, 16, dout, words - 1)  # out too small
    for b in (dq, dout):
        b.close()


@pytest.mark.parametrize("threads", [256, 512, 1024])
@pytest.mark.parametrize("loads", [2, 4, 8])
def test_read_floor_shapes_read_every_byte(ctx, axc, threads, loads):
    """Each launch shape of the read sweep reads exactly the bytes it is given."""
    nbytes = (3 << 20) + 80
    data = np.random.default_rng(threads + loads).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    dq = ctx.alloc(nbytes)
    ctx.upload(dq, data)
    for grid in (1, 256, 2048):
        words = grid * threads // 64
        dout = ctx.alloc(words * 4)
        ctx.read_floor_shape(dq, nbytes, threads, loads, grid, dout, words)
        ctx.synchronize()
        got = np.frombuffer(ctx.download(dout, words * 4), dtype=np.uint32)
        assert int(np.bitwise_xor.reduce(got)) == int(np.bitwise_xor.reduce(data)), grid
        with pytest.raises(axc.DispatchError):
            ctx.read_floor_shape(dq, nbytes, threads, loads, grid, dout, words - 1)
        dout.close()
    with pytest.raises(axc.DispatchError):
        ctx.read_floor_shape(dq, nbytes, 128, loads, 1, dq, 1 << 18)
    with pytest.raises(axc.DispatchError):
        ctx.read_floor_shape(dq, nbytes, threads, 3, 1, dq, 1 << 18)
    with pytest.raises(axc.DispatchError):
        ctx.read_floor_shape(dq, 1 << 32, threads, loads, 1, dq, 1 << 18)
    dq.close()
