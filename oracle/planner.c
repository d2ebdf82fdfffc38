/*
 * Oracle: decoder and encoder KV ring planners (TEST INFRASTRUCTURE ONLY).
 *
 * Restates the integer ring arithmetic of the reference:
 *   decoder: clear_kv_cache / decoder_kv_segments / voxtral_decoder_kv_plan /
 *            decoder_kv_commit_plan   (src/voxtral.cpp:1590-1656)
 *   encoder: voxtral_enc_kv_mask_allows / enc_kv_ring_segments /
 *            voxtral_enc_kv_plan      (src/voxtral.cpp:3636-3692)
 *   encoder run scheduling: normalize_physical_rows (:104-111),
 *            encoder_kv_schedule_from_env (:125-154), enc_frames_realizable
 *            (:3700-3702), encoder_kv_drive (:4379-4426)
 * Pinned by the known-answer vectors of tests/cpp/test_decoder_kv.cpp and
 * tests/cpp/test_encoder_kv.cpp (restated in tests/test_planner.py) and by a
 * brute-force slot->absolute-position ring model; the scheduling by closed
 * forms and by the invariants the reference states for the drive (startup
 * block, full logical batches during feed, no run across a query block, runs
 * independent of the audio chunking), tests/test_enc_drive.py.
 */
#include "vkv_oracle.h"

#include <string.h>

static int64_t orc_min64(int64_t a, int64_t b) { return a < b ? a : b; }
static int64_t orc_max64(int64_t a, int64_t b) { return a > b ? a : b; }

/* Split [abs_start, abs_start+len) into <=2 physical segments.
 * src/voxtral.cpp:1604-1613 (decoder) and :3642-3651 (encoder) are the same rule. */
static int32_t orc_segments(int64_t abs_start, int32_t len, int32_t capacity, orc_seg out[2]) {
    if (len <= 0) return 0;
    int32_t slot = (int32_t)(abs_start % capacity);
    int32_t first = len < capacity - slot ? len : capacity - slot;
    out[0].slot = slot;
    out[0].len = first;
    if (first >= len) return 1;
    out[1].slot = 0;
    out[1].len = len - first;
    return 2;
}

/* src/voxtral.cpp:1615-1644 */
bool orc_decoder_plan(const orc_ring *ring, int64_t absolute_start, int32_t n_new, orc_plan_t *out) {
    memset(out, 0, sizeof(*out));
    if (ring->capacity <= 0 || ring->used < 0 || ring->used > ring->capacity ||
        ring->oldest_absolute_position < 0 || ring->next_absolute_position < 0 ||
        ring->oldest_absolute_position + ring->used != ring->next_absolute_position ||
        absolute_start != ring->next_absolute_position || n_new <= 0 ||
        n_new > ring->capacity) {
        return false;
    }
    out->absolute_start = absolute_start;
    out->n_new = n_new;
    out->write_nseg = orc_segments(absolute_start, n_new, (int32_t)ring->capacity, out->write_seg);
    out->next_after = absolute_start + n_new;
    out->used_after = orc_min64(ring->capacity, ring->used + n_new);
    out->oldest_after = out->next_after - out->used_after;
    out->evicted = orc_max64(0, ring->used + n_new - ring->capacity);
    out->read_nseg = orc_segments(out->oldest_after, (int32_t)out->used_after,
                                  (int32_t)ring->capacity, out->read_seg);
    {
        int64_t previous_cycle = absolute_start == 0 ? 0 : (absolute_start - 1) / ring->capacity;
        int64_t newest_cycle = (out->next_after - 1) / ring->capacity;
        out->wrapped = newest_cycle > previous_cycle;
    }
    return true;
}

/* src/voxtral.cpp:1646-1656 */
void orc_decoder_commit(orc_ring *ring, const orc_plan_t *plan) {
    ring->used = plan->used_after;
    ring->oldest_absolute_position = plan->oldest_after;
    ring->next_absolute_position = plan->next_after;
    ring->evictions += plan->evicted;
    if (plan->wrapped) ring->wraps += 1;
}

/* src/voxtral.cpp:1590-1602: logical invalidation only. */
void orc_decoder_clear(orc_ring *ring, int64_t capacity) {
    memset(ring, 0, sizeof(*ring));
    ring->capacity = capacity;
}

/* src/voxtral.cpp:3636-3638 */
bool orc_enc_mask_allows(int64_t kv_abs, int64_t q_abs, int32_t window) {
    return kv_abs <= q_abs && kv_abs >= q_abs - (int64_t)(window - 1);
}

/* src/voxtral.cpp:3653-3692 */
bool orc_enc_plan(int64_t q_start, int32_t n_new, int32_t capacity, int32_t window,
                  orc_enc_plan_t *out) {
    memset(out, 0, sizeof(*out));
    if (n_new <= 0 || capacity <= 0 || window <= 0) return false;
    if (n_new > capacity - window) return false;
    if (q_start < 0) return false;
    out->q_start = q_start;
    out->n_new = n_new;
    out->win_start = orc_max64(0, q_start - (int64_t)(window - 1));
    out->win_end = q_start + n_new;
    out->win_len = (int32_t)(out->win_end - out->win_start);
    out->read_nseg = orc_segments(out->win_start, out->win_len, capacity, out->read_seg);
    out->read_wraps = out->read_nseg > 1;
    out->write_nseg = orc_segments(q_start, n_new, capacity, out->write_seg);
    out->write_wraps = out->write_nseg > 1;
    out->conv_mel_start = orc_max64(0, 2 * (q_start - 2));
    out->conv_mel_end = 2 * (q_start + n_new);
    out->conv_slice_start = (int32_t)(q_start - out->conv_mel_start / 2);
    {
        int64_t old_lo = orc_max64(0, q_start - (int64_t)window);
        int64_t new_lo = orc_max64(0, out->win_end - (int64_t)window);
        out->evicted = new_lo - old_lo;
    }
    return true;
}

/* src/voxtral.cpp:104-111 */
int32_t orc_enc_normalize_physical(int32_t rows) {
    static const int32_t steps[] = {4, 8, 16, 32, 64};
    for (int i = 0; i < 5; ++i)
        if (rows <= steps[i]) return steps[i];
    return 128;
}

/* src/voxtral.cpp:125-154 */
void orc_enc_schedule(int32_t throughput, int32_t grid, int32_t logical, int32_t physical,
                      int32_t *out_logical, int32_t *out_physical) {
    const int32_t max_new = 128;
    int32_t lg = 4, ph = 4;
    if (throughput) {
        *out_logical = *out_physical = max_new;
        return;
    }
    if (grid > 0) {
        lg = grid < max_new ? grid : max_new;
        if (grid >= 32) ph = orc_enc_normalize_physical(grid);
    }
    if (logical > 0) lg = logical;
    if (lg > max_new) lg = max_new;
    ph = orc_enc_normalize_physical(physical > 0 ? physical : ph);
    if (lg < 1) lg = 1;
    if (lg > ph || ph % lg != 0) {
        if (lg > ph) lg = ph;
        while (lg > 1 && ph % lg != 0) --lg;
    }
    *out_logical = lg;
    *out_physical = ph;
}

/* src/voxtral.cpp:3700-3702 */
int64_t orc_enc_frames_realizable(int64_t mel_frames) {
    if (mel_frames < 2) return 0;
    return (mel_frames - 2) / 2 + 1;
}

/* src/voxtral.cpp:4379-4426: the body of the drive loop once; n = 0 where the
 * loop breaks or ends. */
bool orc_enc_drive_next(int64_t emitted, int64_t target, bool final, int32_t logical,
                        int32_t physical, int32_t finish_physical, bool batch_terminal,
                        orc_enc_run *out) {
    const int32_t max_new = 128;
    memset(out, 0, sizeof(*out));
    if (!(emitted < target)) return true;
    const int64_t rem = target - emitted;
    if (emitted == 0 && !final && target < max_new) return true;
    if (emitted == 0 && target >= max_new) {
        out->q0 = 0;
        out->n = max_new;
        out->physical = max_new;
        out->warmup = 1;
        return true;
    }
    if (!final && rem < logical) return true;
    const bool terminal = final && batch_terminal;
    const int32_t p = terminal ? finish_physical : physical;
    const int32_t lg = terminal ? finish_physical : logical;
    if (p <= 0) return false;
    const int32_t q_offset = (int32_t)(emitted % p);
    int64_t n = lg;
    if (p - q_offset < n) n = p - q_offset;
    if (rem < n) n = rem;
    if (n <= 0) return false;
    out->q0 = emitted;
    out->n = (int32_t)n;
    out->physical = p;
    return true;
}
