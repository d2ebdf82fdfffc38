"""Encoder run scheduling (encoder_kv_drive, src/voxtral.cpp:4379-4426, with
normalize_physical_rows :104-111, encoder_kv_schedule_from_env :125-154 and
enc_frames_realizable :3700-3702): the product's host functions (libvkv.so,
no GPU work) against the oracle's restatement, and both against what the
reference's own comments fix -- the 128-frame startup block, full logical
batches during feed, runs that never cross a physical query block, and a
sequence of runs that does not depend on how the audio was chunked."""
import random

import pytest

import oracle
import vkv

CAP, WIN, MAX_NEW = 878, 750, 128


def test_normalize_physical_closed_form():
    for rows in range(-3, 300):
        want = 4 if rows <= 4 else 8 if rows <= 8 else 16 if rows <= 16 else \
            32 if rows <= 32 else 64 if rows <= 64 else 128
        assert vkv.enc_normalize_physical(rows) == want == oracle.enc_normalize_physical(rows)


@pytest.mark.parametrize("args,want", [
    ((0, 0, 0, 0), (4, 4)),          # defaults
    ((1, 0, 0, 0), (128, 128)),      # VOXTRAL_ENC_KV_MODE=throughput
    ((0, 16, 0, 0), (4, 4)),         # legacy grid below 32: logical-only, clamped to physical
    ((0, 64, 0, 0), (64, 64)),       # legacy grid 64: a full grid
    ((0, 200, 0, 0), (128, 128)),
    ((0, 0, 8, 16), (8, 16)),
    ((0, 0, 3, 8), (2, 8)),          # physical must hold whole logical batches
    ((0, 0, 7, 5), (4, 8)),          # physical 5 -> 8; logical 7 -> 4
    ((0, 0, 500, 0), (4, 4)),        # logical clamps to 128, then to physical 4
    ((0, 48, 12, 0), (8, 64)),       # grid sets physical 64; logical 12 -> 8
])
def test_schedule_make_cases(args, want):
    sc = vkv.enc_schedule(*args)
    assert (sc.logical, sc.physical) == want
    assert oracle.enc_schedule(*args) == want


def test_schedule_make_agrees_everywhere():
    for thr in (0, 1):
        for grid in (0, 1, 3, 16, 31, 32, 33, 64, 100, 128, 129):
            for lg in (0, 1, 2, 3, 4, 5, 8, 12, 16, 64, 127, 128, 300):
                for ph in (0, 1, 4, 5, 8, 9, 16, 32, 33, 64, 65, 128, 400):
                    sc = vkv.enc_schedule(thr, grid, lg, ph)
                    o = oracle.enc_schedule(thr, grid, lg, ph)
                    assert (sc.logical, sc.physical) == o
                    assert sc.physical % sc.logical == 0 and 1 <= sc.logical <= sc.physical


def test_frames_realizable_closed_form():
    for mel in range(-2, 5000):
        want = 0 if mel < 2 else (mel - 2) // 2 + 1
        assert vkv.enc_frames_realizable(mel) == want == oracle.enc_frames_realizable(mel)


def drive(emitted, target, final, sc, finish_physical, batch_terminal):
    """Both implementations, compared on every call; returns the runs until the
    drive stops."""
    runs = []
    while True:
        r = vkv.enc_drive_next(emitted, target, final, sc, finish_physical, batch_terminal)
        o = oracle.enc_drive_next(emitted, target, final, sc.logical, sc.physical,
                                  finish_physical, batch_terminal)
        assert o == (r.q0, r.n, r.physical, r.warmup)
        if r.n == 0:
            return emitted, runs
        assert r.q0 == emitted
        runs.append((r.q0, r.n, r.physical, r.warmup))
        emitted += r.n


def stream(mel_total, right_pad, chunks, sc, finish_physical, batch_terminal):
    emitted, runs, fed, feed_runs = 0, [], 0, 0
    for c in chunks:
        fed += c
        emitted, new = drive(emitted, vkv.enc_frames_realizable(fed), False, sc, finish_physical,
                             batch_terminal)
        runs += new
    assert fed == mel_total
    feed_runs = len(runs)
    target = vkv.enc_frames_realizable(mel_total + right_pad)
    emitted, new = drive(emitted, target, True, sc, finish_physical, batch_terminal)
    runs += new
    return runs, feed_runs, target


def random_chunks(rng, total):
    out = []
    while total > 0:
        c = min(total, rng.choice([1, 2, 3, 8, 17, 80, 160, 333]))
        out.append(c)
        total -= c
    return out


@pytest.mark.parametrize("sched", [(0, 0, 0, 0), (0, 0, 2, 8), (0, 0, 16, 16), (1, 0, 0, 0),
                                   (0, 0, 8, 32)])
@pytest.mark.parametrize("batch_terminal,finish_physical", [(False, 8), (True, 8), (True, 16)])
def test_drive_stream_invariants(sched, batch_terminal, finish_physical):
    rng = random.Random(hash((sched, batch_terminal, finish_physical)) & 0xffff)
    sc = vkv.enc_schedule(*sched)
    for trial in range(40):
        mel_total = rng.choice([0, 1, 2, 50, 255, 256, 257, 300, 1000, 2400, 6001])
        right_pad = rng.choice([0, 72, 144])
        a = stream(mel_total, right_pad, random_chunks(rng, mel_total), sc, finish_physical,
                   batch_terminal)
        b = stream(mel_total, right_pad, random_chunks(rng, mel_total), sc, finish_physical,
                   batch_terminal)
        # the chunking of the audio does not change the runs
        assert a == b
        runs, feed_runs, target = a
        # the runs tile [0, target) in order
        pos = 0
        for i, (q0, n, phys, warm) in enumerate(runs):
            assert q0 == pos and 1 <= n <= MAX_NEW
            assert q0 % phys + n <= phys                    # never crosses a query block
            assert vkv.enc_plan(q0, n, CAP, WIN).n_new == n  # each run is a valid ring plan
            if warm:
                assert i == 0 and (q0, n, phys) == (0, MAX_NEW, MAX_NEW)
            elif i < feed_runs:
                assert n == sc.logical and phys == sc.physical   # full logical batches in feed
            elif batch_terminal:
                assert phys == finish_physical and n <= finish_physical
            else:
                assert phys == sc.physical and n <= sc.logical
            pos += n
        assert pos == target
        # the startup block runs first whenever 128 frames are realizable
        if target >= MAX_NEW:
            assert runs[0] == (0, MAX_NEW, MAX_NEW, 1)
        # nothing runs during feed before the startup block
        if feed_runs:
            assert runs[0][3] == 1


def test_drive_waits_during_feed():
    sc = vkv.enc_schedule()
    # below the startup boundary nothing runs until finish
    r = vkv.enc_drive_next(0, 127, False, sc)
    assert r.n == 0
    r = vkv.enc_drive_next(0, 127, True, sc)
    assert (r.q0, r.n, r.physical, r.warmup) == (0, 4, 4, 0)
    # after the startup block, partial logical batches wait
    sc8 = vkv.enc_schedule(0, 0, 8, 8)
    assert vkv.enc_drive_next(128, 135, False, sc8).n == 0
    r = vkv.enc_drive_next(128, 136, False, sc8)
    assert (r.q0, r.n, r.physical) == (128, 8, 8)
    # finish flushes the remainder, never across a block: 133 % 8 = 5 -> 3 rows fit
    r = vkv.enc_drive_next(133, 140, True, sc8)
    assert (r.q0, r.n, r.physical) == (133, 3, 8)


def test_drive_rejects_bad_arguments():
    bad = vkv.EncSchedule(0, 4)
    with pytest.raises(vkv.VkvError):
        vkv.enc_drive_next(0, 10, True, bad)
    with pytest.raises(vkv.VkvError):
        vkv.enc_drive_next(4, 10, True, vkv.enc_schedule(), finish_physical=0, batch_terminal=True)
    assert oracle.enc_drive_next(4, 10, True, 4, 4, 0, True) is None
