"""GPU: lazily coherent host buffers (gncx_hip_set_host_coherence(1)).

Buffers from gncx_ram_alloc_colored keep a device copy; calls use it in
place and outputs stay on the device until the host touches them (a page
fault brings them back).  Every result must equal the synchronous host-buffer
path bit for bit, through plain numpy / torch reads and writes of the
buffers between calls, partial writes, in-place calls, KV caches, the
4-phase token arrays of the streamer, copies into and frees of buffers the
device holds, and a flush before a system call."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

import synth
from conftest import gncx, ptr, rel_l2

pytestmark = pytest.mark.gpu
Q4_K = 12


@pytest.fixture
def lazy(lib):
    before = lib.gncx_hip_set_host_coherence(1)
    assert before == 0
    handles = []

    def alloc(n, slot=0):
        h = lib.gncx_ram_alloc_colored(max(4 * n, 4096), 1, slot, 3)
        assert h
        handles.append(h)
        return h, np.ctypeslib.as_array((C.c_float * n).from_address(lib.gncx_ram_get_ptr(h)))

    yield alloc
    for h in handles:
        lib.gncx_ram_free(h)
    lib.gncx_hip_set_host_coherence(0)
    lib.gncx_hip_last_status()


def test_lazy_matvec_follows_host_reads_and_writes(lib, oracle, lazy):
    k, n = 1024, 300
    w = synth.make_weights(Q4_K, n, k, seed=61)
    _, x = lazy(k, 1)
    _, y = lazy(n, 2)
    x[:] = synth.make_activations(1, k, seed=62)
    y[:] = 5.0
    for rnd in range(3):
        lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
        gncx.check(lib)
        want = oracle.matvec(Q4_K, w, x.copy(), k, n)
        assert rel_l2(y, want) < 1e-3, rnd          # a host read brings y back
        assert rel_l2(y.copy(), want) < 1e-3        # and reads again without a round trip
        x[::7] *= -1.5                              # a host write to x: the next call uploads it
    # in place on a buffer the device holds, then a partial host write
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
    lib.gncx_hip_vec_add(y.ctypes.data, y.ctypes.data, n)
    gncx.check(lib)
    want = 2 * oracle.matvec(Q4_K, w, x.copy(), k, n)
    assert rel_l2(y, want) < 1e-3
    y[10] = 123.0
    lib.gncx_hip_vec_add(y.ctypes.data, y.ctypes.data, n)
    want[10] = 123.0
    assert rel_l2(y, 2 * want) < 1e-3 and y[10] == 246.0


def test_lazy_adaptive_policies_keep_results_exact(lib, oracle, lazy):
    """Buffers whose use settles into a pattern switch policy: an input the
    host rewrites after every upload keeps read-write pages (and is uploaded
    again for each device read); an output the host reads after every call
    is copied home before the writing call returns (and once every 64 such
    calls goes through the fault path again).  Results stay exact through
    the switches, through calls whose output the host skips, and through
    host writes into a buffer that the device then reads."""
    k, n = 512, 256
    w = synth.make_weights(Q4_K, n, k, seed=71)
    _, x = lazy(k, 1)
    _, y = lazy(n, 2)
    x[:] = synth.make_activations(1, k, seed=72)
    for rnd in range(80):  # past both switch points and one re-check of the copy home
        lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
        gncx.check(lib)
        assert rel_l2(y, oracle.matvec(Q4_K, w, x.copy(), k, n)) < 1e-3, rnd
        x[rnd % k] += 0.25  # rewritten after each upload
    for rnd in range(3):    # outputs the host does not read
        x[::5] *= -1.0
        lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
    gncx.check(lib)
    want = oracle.matvec(Q4_K, w, x.copy(), k, n)
    assert rel_l2(y, want) < 1e-3
    y[:16] = 7.0            # host write into the output, then a device read of it
    want[:16] = 7.0
    lib.gncx_hip_vec_add(y.ctypes.data, y.ctypes.data, n)
    gncx.check(lib)
    assert rel_l2(y, 2 * want) < 1e-3 and np.all(y[:16] == 14.0)


def test_lazy_deferred_matvecs_issue_before_every_consumer(lib, oracle, lazy):
    """Consecutive matvecs on one device-held input are gathered into one
    launch (at most four matrices; a differing input, type or in_dim starts a
    new group).  Every consumer finds them issued: a host read of an output,
    a later device call reading it, and a matvec whose input is a gathered
    output.  Results equal the oracle's."""
    k = 512
    ns = [96, 160, 256, 64, 128]
    ws = [synth.make_weights(Q4_K, n, k, seed=80 + i) for i, n in enumerate(ns)]
    _, x = lazy(k, 1)
    _, xn = lazy(k, 2)
    ys = [lazy(n, 3 + i)[1] for i, n in enumerate(ns)]
    x[:] = synth.make_activations(1, k, seed=90)
    # xn: a device-held input (the output of a device call), as the streamer's normalised vector
    lib.gncx_hip_vec_add(xn.ctypes.data, x.ctypes.data, k)
    for i, w in enumerate(ws):  # five on one input: a group of four, then one more
        lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, xn.ctypes.data, None, k, ns[i], ys[i].ctypes.data, None)
    gncx.check(lib)
    xs = xn.copy()  # host read of the input: every pending matvec is issued first
    for i, w in enumerate(ws):
        assert rel_l2(ys[i], oracle.matvec(Q4_K, w, xs, k, ns[i])) < 1e-3, i
    # gathered outputs (fresh buffers) consumed by a device call, then read on the host
    us = [lazy(ns[i], 10 + i)[1] for i in range(3)]
    for i in range(3):
        lib.gncx_xfold_universal_matvec(ptr(ws[i]), 0, Q4_K, xn.ctypes.data, None, k, ns[i], us[i].ctypes.data, None)
    lib.gncx_hip_vec_add(us[0].ctypes.data, us[0].ctypes.data, ns[0])
    gncx.check(lib)
    assert rel_l2(us[0], 2 * oracle.matvec(Q4_K, ws[0], xs, k, ns[0])) < 1e-3
    assert rel_l2(us[2], oracle.matvec(Q4_K, ws[2], xs, k, ns[2])) < 1e-3
    # a matvec whose input is a gathered output (k = 256 = ns[2])
    wc = synth.make_weights(Q4_K, 64, 256, seed=95)
    _, u3 = lazy(ns[2], 14)
    _, z = lazy(64, 15)
    lib.gncx_xfold_universal_matvec(ptr(ws[2]), 0, Q4_K, xn.ctypes.data, None, k, ns[2], u3.ctypes.data, None)
    lib.gncx_xfold_universal_matvec(ptr(wc), 0, Q4_K, u3.ctypes.data, None, 256, 64, z.ctypes.data, None)
    gncx.check(lib)
    y2 = oracle.matvec(Q4_K, ws[2], xs, k, ns[2])
    assert rel_l2(z, oracle.matvec(Q4_K, wc, y2, 256, 64)) < 1e-3


def test_lazy_weight_rewritten_between_gathered_matvecs(lib, oracle, lazy):
    """A host weight array rewritten in place between two matvecs of one
    gathered group: the second call finds the cached device copy stale and
    replaces it, and the first (still recorded) matvec must have read the old
    weights, not freed memory or the new upload at the same address."""
    k, n = 512, 192
    w = synth.make_weights(Q4_K, n, k, seed=121)
    w_old = w.copy()
    w_new = synth.make_weights(Q4_K, n, k, seed=122)
    _, x = lazy(k, 1)
    _, xn = lazy(k, 2)
    _, y1 = lazy(n, 3)
    _, y2 = lazy(n, 4)
    x[:] = synth.make_activations(1, k, seed=123)
    lib.gncx_hip_vec_add(xn.ctypes.data, x.ctypes.data, k)  # a device-held input
    for rnd in range(2):
        lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, xn.ctypes.data, None, k, n, y1.ctypes.data, None)
        w[:] = w_new if rnd == 0 else w_old  # same address, other contents
        lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, xn.ctypes.data, None, k, n, y2.ctypes.data, None)
        gncx.check(lib)
        xs = xn.copy()
        first, second = (w_old, w_new) if rnd == 0 else (w_new, w_old)
        assert rel_l2(y1, oracle.matvec(Q4_K, first, xs, k, n)) < 1e-3, rnd
        assert rel_l2(y2, oracle.matvec(Q4_K, second, xs, k, n)) < 1e-3, rnd
    lib.gncx_hip_weight_forget(ptr(w))


@pytest.mark.parametrize("interrupt", [False, True])
def test_lazy_deferred_attention_prologue(lib, lazy, interrupt):
    """heads-RMSNorm of q and of k, RoPE of both and the attention step on
    device-held q and k run as the attention kernel's fused prologue in lazy
    mode; q, k and the cache row are left as the separate calls leave them
    (bit for bit) and the output matches.  interrupt: a host read of q after
    its normalisation issues the recorded work as separate kernels."""
    H, KV, hd, ctx = 32, 8, 128, 200
    pos, eps, base, scale = ctx - 1, 1e-6, 1e6, 1 / np.sqrt(hd)
    rng = np.random.default_rng(5)
    q0 = rng.standard_normal(H * hd, dtype=np.float32)
    k0 = rng.standard_normal(KV * hd, dtype=np.float32)
    v0 = rng.standard_normal(KV * hd, dtype=np.float32)
    kc0 = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    vc0 = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    norms = np.concatenate([synth.make_norm_gamma(hd, 1), synth.make_norm_gamma(hd, 2)]).astype(np.float32)

    def run(qh, kh, vh, kch, vch, outh, read_q=None):
        lib.gncx_rmsnorm_inplace_heads(qh, ptr(norms), 0, 1, H, hd, eps)
        if read_q is not None:
            read_q()
        lib.gncx_rmsnorm_inplace_heads(kh, ptr(norms), hd * 4, 1, KV, hd, eps)
        lib.gncx_apply_rope_xor11_ext(qh, kh, None, None, 0, 0, H, KV, hd, pos, base)
        lib.gncx_mqa_attention_step_ext(qh, kh, vh, kch, vch, pos, H, KV, hd, scale, 0, 1, outh)
        gncx.check(lib)

    # synchronous host buffers: the separate kernels
    lib.gncx_hip_set_host_coherence(0)
    try:
        q1, k1, kc1, vc1 = q0.copy(), k0.copy(), kc0.copy(), vc0.copy()
        out1 = np.zeros(H * hd, np.float32)
        run(ptr(q1), ptr(k1), ptr(v0), ptr(kc1), ptr(vc1), ptr(out1))
        lib.gncx_hip_kv_forget(None)
    finally:
        lib.gncx_hip_set_host_coherence(1)
    # lazy buffers, q and k produced on the device
    _, qs = lazy(H * hd, 1)
    _, ks = lazy(KV * hd, 2)
    _, q = lazy(H * hd, 3)
    _, k = lazy(KV * hd, 4)
    _, v = lazy(KV * hd, 5)
    _, kc = lazy(ctx * KV * hd, 6)
    _, vc = lazy(ctx * KV * hd, 7)
    _, out = lazy(H * hd, 8)
    qs[:], ks[:], v[:] = q0, k0, v0
    kc[:], vc[:] = kc0.reshape(-1), vc0.reshape(-1)
    lib.gncx_hip_vec_add(q.ctypes.data, qs.ctypes.data, H * hd)  # q = 0 + q0, device-held
    lib.gncx_hip_vec_add(k.ctypes.data, ks.ctypes.data, KV * hd)
    seen = []
    run(q.ctypes.data, k.ctypes.data, v.ctypes.data, kc.ctypes.data, vc.ctypes.data, out.ctypes.data,
        (lambda: seen.append(q.copy())) if interrupt else None)
    assert np.array_equal(q, q1) and np.array_equal(k, k1)
    assert np.array_equal(kc.reshape(ctx, -1), kc1) and np.array_equal(vc.reshape(ctx, -1), vc1)
    assert rel_l2(out, out1) < 1e-6
    if interrupt:
        q_norm = q0.copy()
        lib.gncx_hip_set_host_coherence(0)
        try:
            lib.gncx_rmsnorm_inplace_heads(ptr(q_norm), ptr(norms), 0, 1, H, hd, eps)
        finally:
            lib.gncx_hip_set_host_coherence(1)
        assert np.array_equal(seen[0], q_norm)
    lib.gncx_hip_kv_forget(None)


def test_lazy_elementwise_outputs_stay_on_device(lib, golden, lazy):
    """SwiGLU and GeGLU chained through lazy buffers, one in place; the
    outputs are read on the host only at the end."""
    gg, uu = golden["swi_g"], golden["swi_u"]
    nf = gg.size
    _, g = lazy(nf, 1)
    _, u = lazy(nf, 2)
    _, a = lazy(nf, 3)
    _, b = lazy(nf, 4)
    g[:], u[:] = gg, uu
    lib.gncx_swiglu_activation(g.ctypes.data, u.ctypes.data, nf, a.ctypes.data)
    lib.gncx_geglu_activation(a.ctypes.data, u.ctypes.data, nf, b.ctypes.data)
    lib.gncx_swiglu_activation(g.ctypes.data, u.ctypes.data, nf, g.ctypes.data)  # in place
    gncx.check(lib)
    lib.gncx_hip_set_host_coherence(0)
    try:
        hg, hu = gg.copy(), uu.copy()  # named: the library reads them during the calls
        ref_a = np.zeros(nf, np.float32)
        ref_b = np.zeros(nf, np.float32)
        lib.gncx_swiglu_activation(ptr(hg), ptr(hu), nf, ptr(ref_a))
        lib.gncx_geglu_activation(ptr(ref_a), ptr(hu), nf, ptr(ref_b))
    finally:
        lib.gncx_hip_set_host_coherence(1)
    assert np.array_equal(b, ref_b)
    assert np.array_equal(a, ref_a)
    assert np.array_equal(g, ref_a)


def test_lazy_flush_before_system_call(lib, oracle, lazy, tmp_path):
    k, n = 512, 1024
    w = synth.make_weights(Q4_K, n, k, seed=63)
    _, x = lazy(k, 1)
    _, y = lazy(n, 2)
    x[:] = synth.make_activations(1, k, seed=64)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
    gncx.check(lib)
    lib.gncx_hip_host_flush(y.ctypes.data)
    f = tmp_path / "y.bin"
    fd = os.open(f, os.O_WRONLY | os.O_CREAT)
    try:
        assert os.write(fd, memoryview(y).cast("B")) == 4 * n
    finally:
        os.close(fd)
    assert rel_l2(np.fromfile(f, np.float32), oracle.matvec(Q4_K, w, x.copy(), k, n)) < 1e-3


def test_lazy_copy_chunk_and_free_of_device_held_buffers(lib, oracle, lazy):
    k, n = 512, 256
    w = synth.make_weights(Q4_K, n, k, seed=65)
    _, x = lazy(k, 1)
    hy, y = lazy(n, 2)
    x[:] = synth.make_activations(1, k, seed=66)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
    gncx.check(lib)
    src = np.arange(16, dtype=np.float32)
    lib.gncx_ram_copy_chunk(hy, 8, ptr(src), 0, src.nbytes)   # into a buffer the device holds
    want = oracle.matvec(Q4_K, w, x.copy(), k, n)
    want[2:18] = src
    assert rel_l2(y, want) < 1e-3 and np.array_equal(y[2:18], src)
    # freeing a buffer whose newest data is on the device
    h2 = lib.gncx_ram_alloc_colored(4 * n, 2, 3, 5)
    y2 = np.ctypeslib.as_array((C.c_float * n).from_address(lib.gncx_ram_get_ptr(h2)))
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y2.ctypes.data, None)
    del y2
    lib.gncx_ram_free(h2)
    gncx.check(lib)


def test_lazy_decode_equals_synchronous_host_buffers(lib, torch_mod, tmp_path):
    """The streamer's decode through buffers from gncx_ram_alloc_colored and
    the 4-phase token array, with lazy coherence and without, issued from
    Python and from the native replay of forward_token: identical logits,
    token arrays and KV caches."""
    import gncx_amd.decode as dec
    from test_gpu_decode import small_shape
    dec.write_model_gguf(tmp_path / "m.gguf", small_shape(), seed=34)
    m = dec.load_model_gguf(tmp_path / "m.gguf")
    runs = []
    try:
        for lazy_mode, driver in ((0, "python"), (1, "python"), (0, "c"), (1, "c")):
            lib.gncx_hip_set_host_coherence(lazy_mode)
            d = dec.Decoder(lib, torch_mod, m, max_seq=16, device="cpu", host="ram", tokens=True, driver=driver)
            try:
                tok, logits, toks = 11, [], []
                for pos in range(6):
                    a = d.forward_token(tok, pos).numpy().copy()
                    gncx.check(lib)
                    logits.append(a)
                    toks.append(bytes(d.tokens))
                    tok = d.greedy(d.logits)
                kc = d.kc[1].numpy()[:6].copy()
                vc = d.vc[0].numpy()[:6].copy()
                runs.append((logits, toks, kc, vc))
            finally:
                lib.gncx_hip_set_host_coherence(0)
                d.close()
        la, ta, ka, va = runs[0]
        assert np.abs(ka).sum() > 0
        for r, (lb, tb, kb, vb) in enumerate(runs[1:], 1):
            for i in range(len(la)):
                assert np.array_equal(la[i], lb[i]), (r, i)
                assert ta[i] == tb[i], (r, i)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), r
    finally:
        lib.gncx_hip_set_host_coherence(0)
        lib.gncx_hip_weight_forget(None)
        lib.gncx_hip_kv_forget(None)


def test_lazy_fault_inside_lock_holding_libc_call(lib, oracle, lazy, tmp_path):
    """The first host access to a buffer the device holds happens inside
    fwrite, which holds the stream's lock while it copies the bytes into its
    own buffer (1200 bytes: below the stdio buffer, so the copy is a user-space
    read that faults, not a write(2) that would fail with EFAULT).  The fault
    is resolved by the library's resolver thread, not in the handler, and the
    file holds the device's result."""
    k, n = 512, 300
    w = synth.make_weights(Q4_K, n, k, seed=71)
    _, x = lazy(k, 1)
    _, y = lazy(n, 2)
    x[:] = synth.make_activations(1, k, seed=72)
    want = oracle.matvec(Q4_K, w, x.copy(), k, n)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
    gncx.check(lib)
    libc = C.CDLL(None)
    libc.fopen.restype = C.c_void_p
    libc.fopen.argtypes = [C.c_char_p, C.c_char_p]
    libc.fwrite.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
    libc.fclose.argtypes = [C.c_void_p]
    path = tmp_path / "y.bin"
    fp = libc.fopen(str(path).encode(), b"wb")
    assert fp
    assert libc.fwrite(y.ctypes.data, 4, n, fp) == n
    assert libc.fclose(fp) == 0
    got = np.fromfile(path, dtype=np.float32)
    assert rel_l2(got, want) < 1e-3
    assert np.array_equal(got, y)


def test_lazy_fault_while_another_thread_calls_the_library(lib, oracle, lazy):
    """A host read of a device-held buffer faults while another thread keeps
    the library busy with synchronous calls of its own: the resolver waits
    its turn for the call lock like any call, nothing deadlocks, and both
    threads get correct results."""
    import threading

    k, n = 1024, 400
    w = synth.make_weights(Q4_K, n, k, seed=73)
    _, x = lazy(k, 1)
    _, y = lazy(n, 2)
    x[:] = synth.make_activations(1, k, seed=74)
    want = oracle.matvec(Q4_K, w, x.copy(), k, n)
    w2 = synth.make_weights(Q4_K, 256, 2048, seed=75)
    x2 = synth.make_activations(1, 2048, seed=76)
    want2 = oracle.matvec(Q4_K, w2, x2, 2048, 256)
    errs = []

    def busy():
        y2 = np.zeros(256, np.float32)  # ordinary host memory: every call waits for its result
        for _ in range(200):
            lib.gncx_xfold_universal_matvec(ptr(w2), 0, Q4_K, ptr(x2), None, 2048, 256, ptr(y2), None)
            errs.append(rel_l2(y2, want2))

    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, x.ctypes.data, None, k, n, y.ctypes.data, None)
    gncx.check(lib)
    t = threading.Thread(target=busy)
    t.start()
    got = y.copy()  # faults while busy() calls the library
    t.join(timeout=60)
    assert not t.is_alive()
    gncx.check(lib)
    assert rel_l2(got, want) < 1e-3
    assert len(errs) == 200 and max(errs) < 1e-3
    lib.gncx_hip_weight_forget(ptr(w2))
