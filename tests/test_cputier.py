"""The host-CPU expert tier (hecate_amd/csrc/cputier.cpp) driven from the host through a plain-memory mailbox, as
tools/dev/test_grace_picks.py drives cpuband's flags: bit-exact against the oracle's q8_0 mode (cpuband.cpp's
arithmetic), a many-pick job equal to the sum of its one-pick jobs (test_grace_picks.py:95-152), the same bits for
any thread count and for either dot kernel (AVX2, AVX-512 VNNI), and the error words of bad jobs. No GPU."""
import numpy as np
import pytest

import pyoracle as O
from hecate_amd.cpu_tier import CpuTier
from hostref import HostLayer, x_rows

LO, N = 248, 8                      # the cold window: ids 248..255 (local id = id - LO, as in a resident bank)


@pytest.fixture(scope="module")
def hl():
    return HostLayer(0, shared=False)


@pytest.fixture(scope="module")
def cold(hl):
    # the tier's local expert e is the host layer's local expert e (the window convention of the banks)
    return [hl.expert(e) for e in range(N)]


def start(cold, threads):
    t = CpuTier(threads=threads, mapped=False)
    t.add_layer(0, LO, cold)
    return t


def picks(R, seed):
    """sel with 3 picks per row in the window (some shared between rows), the rest outside it; f16 weights"""
    rng = np.random.default_rng(seed)
    sel = np.stack([rng.choice(LO, 8, replace=False) for _ in range(R)]).astype(np.int64)
    for r in range(R):
        sel[r, rng.choice(8, 3, replace=False)] = LO + rng.choice(N, 3, replace=False)
    rw = O.f32_to_f16((rng.random((R, 8)) * 0.5 + 0.05).astype(np.float32))
    return sel, rw


def oracle_q8(hl, x, sel, rw):
    return O.moe(1, x, sel, rw, hl.table(sel, LO), LO, N, None, threads=8)


@pytest.mark.parametrize("R", [1, 3, 8])
def test_cpu_tier_matches_oracle_q8(hl, cold, R):
    t = start(cold, 4)
    try:
        x = x_rows(500 + R, R)
        sel, rw = picks(R, R)
        t.post(x, sel, rw, 0)
        out, err = t.wait()
        assert err == 0
        ref = oracle_q8(hl, x, sel, rw)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        assert t.stats()[0] == 1
    finally:
        t.close()


def test_cpu_tier_job_is_sum_of_one_pick_jobs(hl, cold):
    """a job with several cold picks equals the sum, in pick order from 0, of the jobs that keep one of them"""
    t = start(cold, 4)
    try:
        R = 4
        x = x_rows(77, R)
        sel, rw = picks(R, 9)
        t.post(x, sel, rw, 0)
        full, _ = t.wait()
        order = []                                   # pick order: first appearance over rows, then top-k
        for e in sel.ravel():
            if LO <= e < LO + N and e not in order:
                order.append(int(e))
        acc = np.zeros((R, 6144), np.float32)
        for e in order:
            s1 = np.where((sel >= LO) & (sel != e), 0, sel)      # the other cold picks moved out of the window
            t.post(x, s1, rw, 0)
            part, _ = t.wait()
            acc = acc + part
        assert np.array_equal(full.view(np.uint32), acc.view(np.uint32))
    finally:
        t.close()


def test_cpu_tier_thread_count_does_not_change_bits(cold):
    R = 5
    x = x_rows(31, R)
    sel, rw = picks(R, 4)
    outs = []
    for threads in (1, 3, 8):
        t = start(cold, threads)
        try:
            t.post(x, sel, rw, 0)
            outs.append(t.wait()[0])
        finally:
            t.close()
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs[1:])


def test_cpu_tier_bad_jobs(cold):
    t = start(cold, 2)
    try:
        x = x_rows(3, 2)
        sel, rw = picks(2, 1)
        t.post(x, sel, rw, 5)                        # a layer the pool does not hold
        out, err = t.wait()
        assert err == 2 and not out.any()
        t.post(x, sel, rw, 0)                        # and the pool still serves the next job
        _, err = t.wait()
        assert err == 0
        t.mb.rows, t.mb.err = 9, 0                   # a row count past the mailbox
        t.raise_issue(1)
        _, err = t.wait()
        assert err == 1
    finally:
        t.close()


def test_cpu_tier_dot_kernels_agree(cold, monkeypatch):
    """the AVX2 dot and the AVX-512 VNNI dot (taken when the host has it) give the same bits: the same integer lane
    sums reach the same float order (HMOE_CPU_ISA=avx2 forces the first at pool start)"""
    R = 6
    x = x_rows(41, R)
    sel, rw = picks(R, 13)
    outs = []
    for isa in ("avx2", None):
        if isa:
            monkeypatch.setenv("HMOE_CPU_ISA", isa)
        else:
            monkeypatch.delenv("HMOE_CPU_ISA", raising=False)
        t = start(cold, 3)
        try:
            t.post(x, sel, rw, 0)
            outs.append(t.wait()[0])
        finally:
            t.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_cpu_tier_entry_points_reject_bad_arguments(cold):
    """the C ABI's checks (before any GPU call): one pool per process, thread counts, layer shapes, the hand-off's
    row counts and alignment; each failure returns an error code with a message"""
    import ctypes
    from hecate_amd import _lib
    L = _lib.lib()
    mb = (ctypes.c_uint8 * 200_000)()
    assert L.hmoe_cpu_stats(None, None) != 0 and b"no pool" in L.hmoe_last_error()
    assert L.hmoe_cpu_add_layer(0, 0, 0, None, None) != 0
    assert L.hmoe_cpu_start(ctypes.addressof(mb), 0, -1) != 0 and b"threads" in L.hmoe_last_error()
    t = start(cold, 2)
    try:
        assert L.hmoe_cpu_start(ctypes.addressof(mb), 2, -1) != 0 and b"running" in L.hmoe_last_error()
        assert L.hmoe_cpu_add_layer(1, 0, 300, None, None) != 0 and b"arguments" in L.hmoe_last_error()
        buf = np.zeros(1 << 16, np.uint8)
        p = buf.ctypes.data
        # rows past the mailbox, a null pointer, a misaligned one: refused before anything is queued
        assert L.hmoe_cpu_submit(t.addr, p, p, p, 9, 0, None) != 0 and b"rows" in L.hmoe_last_error()
        assert L.hmoe_cpu_submit(t.addr, None, p, p, 1, 0, None) != 0
        assert L.hmoe_cpu_submit(t.addr, p + 2, p, p, 1, 0, None) != 0 and b"aligned" in L.hmoe_last_error()
        assert L.hmoe_cpu_collect(t.addr, p, 0, None) != 0
        assert L.hmoe_cpu_collect(t.addr, p + 4, 1, None) != 0
    finally:
        t.close()
    assert L.hmoe_cpu_stop() == 0                                # (stopping twice is harmless)


# ---- the hand-off protocol under forced timing (tools/dev/test_grace_picks.py:95-152 style, host-driven, no GPU) ----

def test_immediate_repost_while_a_worker_is_held(hl, cold, monkeypatch):
    """pool thread 1 sleeps after every job (HMOE_CPU_HOLD), so each next job is posted while it has not yet looked
    for work: with a 0/1 flag that thread could take the re-raised flag for the job it had just finished and deadlock
    the pool; with generations every job runs once, in order, with the oracle's bits"""
    monkeypatch.setenv("HMOE_CPU_HOLD", "1,30000")
    t = start(cold, 4)
    try:
        for j in range(6):
            R = 1 + j % 3
            x = x_rows(900 + j, R)
            sel, rw = picks(R, 40 + j)
            g = t.post(x, sel, rw, 0)
            out, err = t.wait(timeout=20.0)
            assert err == 0 and int(t.mb.done) == g
            assert np.array_equal(out.view(np.uint32), oracle_q8(hl, x, sel, rw).view(np.uint32)), j
        assert t.stats()[0] == 6
    finally:
        t.close()


def test_stale_done_never_ends_a_wait(hl, cold, monkeypatch):
    """a value of done that is not the posted generation (here a larger stale one, which a '>=' wait would take, as
    the reference's reset of CPU_DONE to 0 guards against, tier_split.py:128-138) does not end the wait: the waiter
    gets the job's own result once the pool finishes it"""
    monkeypatch.setenv("HMOE_CPU_HOLD", "1,300000")        # job 2 waits ~0.3 s for thread 1
    t = start(cold, 3)
    try:
        x = x_rows(60, 2)
        sel, rw = picks(2, 60)
        t.post(x, sel, rw, 0)
        t.wait(timeout=20.0)
        x2 = x_rows(61, 3)
        sel2, rw2 = picks(3, 61)
        g = t.post(x2, sel2, rw2, 0)
        t.mb.done = g + 7                                    # stale, larger than the posted generation
        out, err = t.wait(timeout=20.0)
        assert err == 0 and int(t.mb.done) == g
        assert np.array_equal(out.view(np.uint32), oracle_q8(hl, x2, sel2, rw2).view(np.uint32))
    finally:
        t.close()


def test_stop_during_a_stuck_job(cold, monkeypatch):
    """a job that cannot finish (one thread held for 30 s, the others waiting for it at the job's first barrier) does
    not keep hmoe_cpu_stop from returning: barriers and the hold watch the stop flag"""
    import time
    monkeypatch.setenv("HMOE_CPU_HOLD", "1,30000000")
    t = start(cold, 3)
    x = x_rows(70, 1)
    sel, rw = picks(1, 70)
    t.post(x, sel, rw, 0)
    t.wait(timeout=20.0)                                     # job 1 done; thread 1 now held
    g = t.post(x, sel, rw, 0)                                # job 2: stuck at its first barrier
    time.sleep(0.2)
    assert int(t.mb.done) != g
    t0 = time.perf_counter()
    t.close()
    assert time.perf_counter() - t0 < 5.0


def test_skip_mode_acknowledges_with_zero(cold, monkeypatch):
    """HMOE_CPU_SKIP=1 (cpuband.cpp:40,249's EXL3_TIER_CPU_SKIP): jobs are acknowledged with a zero partial"""
    monkeypatch.setenv("HMOE_CPU_SKIP", "1")
    t = start(cold, 2)
    try:
        x = x_rows(80, 4)
        sel, rw = picks(4, 80)
        t.mb.out[0] = 5.0
        t.post(x, sel, rw, 0)
        out, err = t.wait(timeout=20.0)
        assert err == 0 and not out.any()
    finally:
        t.close()


def test_add_layer_refusal_leaves_the_layer(hl, cold):
    """a call with a null matrix pointer is refused before the layer changes: the pool still serves the old one"""
    import ctypes
    from hecate_amd import _lib
    t = start(cold, 2)
    try:
        n = 2
        q = (ctypes.c_void_p * (3 * n))()
        s = (ctypes.c_void_p * (3 * n))()
        keep = np.zeros(16, np.uint8)
        for i in range(3 * n):
            q[i] = s[i] = keep.ctypes.data
        q[4] = None
        assert _lib.lib().hmoe_cpu_add_layer(0, 0, n, q, s) != 0 and b"null matrix" in _lib.lib().hmoe_last_error()
        x = x_rows(90, 2)
        sel, rw = picks(2, 90)
        t.post(x, sel, rw, 0)
        out, err = t.wait(timeout=20.0)
        assert err == 0 and np.array_equal(out.view(np.uint32), oracle_q8(hl, x, sel, rw).view(np.uint32))
    finally:
        t.close()


def test_cpu_tier_layers_added_while_jobs_run(hl, cold):
    """layers published to a serving pool (ids other than the job's, and the job's own id again with the same
    experts) while jobs run back to back: every job keeps the oracle's bits (the pool reads a layer through one
    atomically published, unchanging record, so a concurrent add never resizes or rewrites what a job reads)"""
    import threading
    t = start(cold, 4)
    try:
        R = 3
        x = x_rows(909, R)
        sel, rw = picks(R, 21)
        ref = oracle_q8(hl, x, sel, rw)
        done = threading.Event()
        added = [0]

        def adder():
            k = 1
            while not done.is_set():
                try:
                    t.add_layer(k % 50 + 1, LO, cold)         # refused while a job is in flight, else published
                    added[0] += 1
                except RuntimeError:
                    pass
                k += 1
        th = threading.Thread(target=adder)
        th.start()
        try:
            for _ in range(40):
                t.post(x, sel, rw, 0)
                out, err = t.wait()
                assert err == 0 and np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        finally:
            done.set()
            th.join()
        assert added[0] > 0
    finally:
        t.close()
