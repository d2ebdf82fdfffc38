"""Uniform adapters over the two planner implementations under test: the
oracle's C restatement (oracle/planner.c) and the product's C++ planners
(libvkv.so, host-only entry points -- no GPU needed)."""
import ctypes

import oracle
import vkv


def _plan_dict(p, segs_of):
    return {
        "absolute_start": p.absolute_start, "n_new": p.n_new,
        "write": segs_of(p.write_seg, p.write_nseg), "read": segs_of(p.read_seg, p.read_nseg),
        "used_after": p.used_after, "oldest_after": p.oldest_after, "next_after": p.next_after,
        "evicted": p.evicted, "wrapped": bool(p.wrapped),
    }


def _enc_dict(p, segs_of):
    return {
        "q_start": p.q_start, "n_new": p.n_new, "win_start": p.win_start, "win_end": p.win_end,
        "win_len": p.win_len, "read": segs_of(p.read_seg, p.read_nseg),
        "read_wraps": bool(p.read_wraps), "write": segs_of(p.write_seg, p.write_nseg),
        "write_wraps": bool(p.write_wraps), "conv_mel_start": p.conv_mel_start,
        "conv_mel_end": p.conv_mel_end, "conv_slice_start": p.conv_slice_start,
        "evicted": p.evicted,
    }


class OraclePlanner:
    name = "oracle"

    def ring(self, capacity, used=0, oldest=0, next_=0):
        r = oracle.new_ring(capacity)
        r.used, r.oldest_absolute_position, r.next_absolute_position = used, oldest, next_
        return r

    def plan(self, ring, start, n):
        p = oracle.decoder_plan(ring, start, n)
        return None if p is None else (p, _plan_dict(p, oracle.segs_of))

    def commit(self, ring, p):
        oracle.decoder_commit(ring, p)

    def enc_plan(self, q, n, cap, win):
        p = oracle.enc_plan(q, n, cap, win)
        return None if p is None else _enc_dict(p, oracle.segs_of)

    def mask(self, kv, q, win):
        return oracle.enc_mask_allows(kv, q, win)


class ProductPlanner:
    name = "product"

    def ring(self, capacity, used=0, oldest=0, next_=0):
        r = vkv.new_ring(capacity)
        r.used, r.oldest_absolute_position, r.next_absolute_position = used, oldest, next_
        return r

    def plan(self, ring, start, n):
        p = vkv.Plan()
        st = vkv.lib.vkv_decoder_plan(ctypes.byref(ring), start, n, ctypes.byref(p))
        if st != vkv.OK:
            assert st == vkv.INVALID_ARGUMENT
            return None
        return p, _plan_dict(p, vkv.plan_segs)

    def commit(self, ring, p):
        vkv.decoder_commit(ring, p)

    def enc_plan(self, q, n, cap, win):
        p = vkv.EncPlan()
        st = vkv.lib.vkv_enc_plan_build(q, n, cap, win, ctypes.byref(p))
        if st != vkv.OK:
            assert st == vkv.INVALID_ARGUMENT
            return None
        return _enc_dict(p, vkv.plan_segs)

    def mask(self, kv, q, win):
        return vkv.enc_mask_allows(kv, q, win)


IMPLS = [OraclePlanner(), ProductPlanner()]
