"""Ring planners: known-answer vectors of the reference's planner tests
(tests/cpp/test_decoder_kv.cpp, tests/cpp/test_encoder_kv.cpp) and the
reference's ground-truth ring-model method, applied to both the oracle's C
restatement and the product's C++ planners.  CPU only."""
import json
import os
import random

import pytest

from planner_impls import IMPLS

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "planner_kat.json")))


def _ring(impl, d):
    return impl.ring(d["capacity"], d["used"], d["oldest"], d["next"])


def logical_positions(plan_d, capacity):
    """Recover, for every read slot, the unique absolute position in
    [oldest_after, next_after) stored there (test_decoder_kv.cpp:32-45)."""
    out = []
    for slot0, n in plan_d["read"]:
        for i in range(n):
            slot = slot0 + i
            for a in range(plan_d["oldest_after"], plan_d["next_after"]):
                if a % capacity == slot:
                    out.append(a)
                    break
    return out


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
class TestDecoderPlanner:
    def test_initial_and_contiguous(self, impl):
        k = KAT["decoder"]["initial_and_contiguous"]
        ring = _ring(impl, k["ring"])
        p, d = impl.plan(ring, k["start"], k["n_new"])
        for key in ("write", "read"):
            assert d[key] == [tuple(s) for s in k[key]]
        for key in ("used_after", "oldest_after", "next_after", "evicted", "wrapped"):
            assert d[key] == k[key], key
        impl.commit(ring, p)
        assert ring.used == 3 and ring.next_absolute_position == 3

    def test_straddled_write_and_logical_read(self, impl):
        k = KAT["decoder"]["straddled_write"]
        ring = _ring(impl, k["ring"])
        _, d = impl.plan(ring, k["start"], k["n_new"])
        for key in ("write", "read"):
            assert d[key] == [tuple(s) for s in k[key]]
        for key in ("used_after", "oldest_after", "next_after", "evicted", "wrapped"):
            assert d[key] == k[key], key
        assert logical_positions(d, 8) == k["logical_positions"]

    def test_single_step_rollover_and_eviction(self, impl):
        k = KAT["decoder"]["single_step_rollover"]
        cap = k["capacity"]
        ring = impl.ring(cap)
        physical = [-1] * cap
        for pos in range(k["steps"]):
            p, d = impl.plan(ring, pos, 1)
            physical[d["write"][0][0]] = pos
            impl.commit(ring, p)
            assert ring.next_absolute_position == pos + 1
            assert ring.used == (pos + 1 if pos < 7 else 8)
            assert ring.oldest_absolute_position == (0 if pos < 8 else pos - 7)
            logical = logical_positions(d, cap)
            assert len(logical) == ring.used
            for i, a in enumerate(logical):
                assert a == ring.oldest_absolute_position + i
                assert physical[a % cap] == a
        f = k["final"]
        assert ring.wraps == f["wraps"]
        assert ring.evictions == f["evictions"]
        assert ring.bytes_moved == f["bytes_moved"] and ring.full_buffer_moves == f["full_buffer_moves"]
        assert ring.oldest_absolute_position == f["oldest"]

    def test_invalid_plans(self, impl):
        for case in KAT["decoder"]["invalid"]["cases"]:
            ring = _ring(impl, case["ring"])
            assert impl.plan(ring, case["start"], case["n_new"]) is None, case["why"]

    def test_longform_metadata_closed_form(self, impl):
        k = KAT["decoder"]["longform_8192"]
        cap = k["capacity"]
        ring = impl.ring(cap)
        checks = {int(s): v for s, v in k["after_step"].items()}
        for pos in range(max(checks) + 1):
            p, _ = impl.plan(ring, pos, 1)
            impl.commit(ring, p)
            if pos in checks:
                want = checks[pos]
                assert ring.used == want["used"]
                assert ring.oldest_absolute_position == want["oldest"]
                assert ring.next_absolute_position == want["next"]
                assert ring.wraps == want["wraps"]
                assert ring.evictions == want["evictions"]
                assert ring.bytes_moved == 0

    def test_bruteforce_ring_model(self, impl):
        """Random multi-token batches on small capacities against a slot->abs
        ground-truth model (the reference's RingModel method)."""
        rng = random.Random(1234)
        for cap in (1, 2, 3, 8, 64, 100):
            ring = impl.ring(cap)
            slots = [-1] * cap
            pos = 0
            wraps = evictions = 0
            for _ in range(300):
                n = rng.randint(1, cap)
                p, d = impl.plan(ring, pos, n)
                # write segments lay [pos, pos+n) down at abs % cap
                a = pos
                for s0, ln in d["write"]:
                    for i in range(ln):
                        assert s0 + i == a % cap
                        slots[s0 + i] = a
                        a += 1
                assert a == pos + n
                used_after = min(cap, ring.used + n)
                assert d["used_after"] == used_after
                assert d["oldest_after"] == pos + n - used_after
                assert d["evicted"] == max(0, ring.used + n - cap)
                prev_cycle = 0 if pos == 0 else (pos - 1) // cap
                assert d["wrapped"] == ((pos + n - 1) // cap > prev_cycle)
                # read segments enumerate the retained window oldest->newest
                expect = list(range(d["oldest_after"], d["next_after"]))
                got = []
                for s0, ln in d["read"]:
                    got.extend(slots[s0:s0 + ln])
                assert got == expect
                wraps += d["wrapped"]
                evictions += d["evicted"]
                impl.commit(ring, p)
                pos += n
            assert ring.wraps == wraps and ring.evictions == evictions


class RingModel:
    """slot -> absolute frame (tests/cpp/test_encoder_kv.cpp:60-80)."""

    def __init__(self, cap):
        self.slot = [-1] * cap
        self.cap = cap

    def apply_writes(self, p):
        a = p["q_start"]
        for s0, ln in p["write"]:
            for i in range(ln):
                self.slot[s0 + i] = a
                a += 1


def verify_plan(p, m, cap):
    """tests/cpp/test_encoder_kv.cpp:82-111"""
    wabs, wtotal = p["q_start"], 0
    for s0, ln in p["write"]:
        for i in range(ln):
            assert 0 <= s0 + i < cap and s0 + i == wabs % cap
            wabs += 1
            wtotal += 1
    assert wtotal == p["n_new"]
    rabs, rtotal = p["win_start"], 0
    for s0, ln in p["read"]:
        for i in range(ln):
            slot = s0 + i
            assert 0 <= slot < cap and rabs % cap == slot
            assert m.slot[slot] == rabs
            rabs += 1
            rtotal += 1
    assert rtotal == p["win_len"] and rabs == p["win_end"]


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
class TestEncoderPlanner:
    E = KAT["encoder"]
    CAP, WIN, MAXNEW = E["capacity"], E["window"], E["max_new"]

    def simulate(self, impl, batches):
        m = RingModel(self.CAP)
        head = 0
        total_evicted = 0
        for n in batches:
            p = impl.enc_plan(head, n, self.CAP, self.WIN)
            assert p is not None
            assert p["win_len"] <= self.WIN - 1 + n and p["win_len"] <= self.CAP
            assert 1 <= len(p["read"]) <= 2 and 1 <= len(p["write"]) <= 2
            m.apply_writes(p)
            verify_plan(p, m, self.CAP)
            total_evicted += p["evicted"]
            head += n
            logical = head - max(0, head - self.WIN)
            assert logical <= self.WIN
            assert head - total_evicted == logical
        return head

    def test_metadata(self, impl):
        assert self.WIN == 750 and self.CAP == self.WIN + self.MAXNEW

    def test_overflow_guards(self, impl):
        for q, n, ok in self.E["overflow_guards"]["cases"]:
            assert (impl.enc_plan(q, n, self.CAP, self.WIN) is not None) == ok, (q, n)

    def test_first_batch(self, impl):
        k = self.E["first_batch"]
        p = impl.enc_plan(k["q_start"], k["n_new"], self.CAP, self.WIN)
        for key in ("win_start", "win_end", "win_len", "read_wraps", "write_wraps",
                    "conv_mel_start", "conv_mel_end", "conv_slice_start", "evicted"):
            assert p[key] == k[key], key
        assert p["read"] == [tuple(s) for s in k["read"]]

    def test_multi_frame_and_steady_state(self, impl):
        s = self.E["simulations"]
        self.simulate(impl, [1] * s["single_4000"][1])
        self.simulate(impl, [4] * s["steady_1000x4"][1])
        self.simulate(impl, [self.MAXNEW] * s["max_new_200"][1])
        self.simulate(impl, [1 + (i * 37) % self.MAXNEW for i in range(500)])

    def test_window_boundary_positions(self, impl):
        k = self.E["window_boundary"]
        for head in k["heads"]:
            for n in k["n_new"]:
                m = RingModel(self.CAP)
                for a in range(max(0, head - self.WIN), head):
                    m.slot[a % self.CAP] = a
                p = impl.enc_plan(head, n, self.CAP, self.WIN)
                m.apply_writes(p)
                verify_plan(p, m, self.CAP)
                assert p["win_start"] == max(0, head - (self.WIN - 1))

    def test_absolute_positions_after_rollover(self, impl):
        p0 = impl.enc_plan(0, 1, self.CAP, self.WIN)
        p1 = impl.enc_plan(self.CAP, 1, self.CAP, self.WIN)
        assert p0["write"][0][0] == p1["write"][0][0]
        assert p0["q_start"] != p1["q_start"] and p1["q_start"] == self.CAP
        for pos in self.E["rollover_slots"]["positions"]:
            assert impl.enc_plan(pos, 1, self.CAP, self.WIN)["write"][0][0] == pos % self.CAP

    def test_wrap_segments(self, impl):
        k = self.E["wrap_segments"]
        head = k["head"]
        m = RingModel(self.CAP)
        for a in range(max(0, head - self.WIN), head):
            m.slot[a % self.CAP] = a
        p = impl.enc_plan(head, k["n_new"], self.CAP, self.WIN)
        assert p["write_wraps"] and p["write"] == [tuple(s) for s in k["write"]]
        m.apply_writes(p)
        verify_plan(p, m, self.CAP)
        assert p["read_wraps"] == k["read_wraps"]

    def test_mask_predicate(self, impl):
        k = self.E["mask"]
        for kv, q, ok in k["cases"]:
            assert impl.mask(kv, q, self.WIN) == ok
        for q in k["batch_q"]:
            ws = max(0, q - (self.WIN - 1))
            for kv in range(ws, q + 1):
                assert impl.mask(kv, q, self.WIN)
            assert not impl.mask(ws - 1, q, self.WIN)
            assert not impl.mask(q + 1, q, self.WIN)

    def test_conv_window_alignment(self, impl):
        k = self.E["conv_alignment"]
        n = k["n_new"]
        for P in k["heads"]:
            p = impl.enc_plan(P, n, self.CAP, self.WIN)
            assert p["conv_mel_start"] % 2 == 0 and p["conv_mel_start"] >= 0
            assert p["conv_mel_end"] == 2 * (P + n)
            assert p["conv_slice_start"] + p["conv_mel_start"] // 2 == P
            if P >= 2:
                assert p["conv_slice_start"] == 2
            else:
                assert p["conv_mel_start"] == 0 and p["conv_slice_start"] == P

    def test_batch_segmentation(self, impl):
        remaining = self.E["batch_segmentation"]["frames"]
        batches = []
        while remaining > 0:
            batches.append(min(self.MAXNEW, remaining))
            remaining -= batches[-1]
        assert self.simulate(impl, batches) == 5000


def test_impls_agree_on_random_plans():
    """Oracle and product planners agree field for field on random inputs,
    including the invalid ones."""
    rng = random.Random(99)
    o, p = IMPLS
    for _ in range(3000):
        cap = rng.choice([1, 5, 8, 64, 878, 8192])
        used = rng.randint(0, cap)
        oldest = rng.randint(0, 10 ** 6)
        nxt = oldest + used + rng.choice([0, 0, 0, 1, -1])
        start = nxt + rng.choice([0, 0, 0, 1])
        n = rng.randint(-1, cap + 1)
        r1, r2 = o.ring(cap, used, oldest, nxt), p.ring(cap, used, oldest, nxt)
        a, b = o.plan(r1, start, n), p.plan(r2, start, n)
        assert (a is None) == (b is None)
        if a is not None:
            assert a[1] == b[1]
        q = rng.randint(-2, 10 ** 6)
        n = rng.randint(-1, 130)
        assert o.enc_plan(q, n, 878, 750) == p.enc_plan(q, n, 878, 750)
