/*
 * l2_model.c — L2 traffic model of the SpMM kernel (measurement infrastructure, used by bench.py).
 *
 * Replays the cache-line accesses of spmmInt8Kernel128/256 on one MI355X XCD through a
 * set-associative L2 and counts the misses of each stream. The kernel's schedule is modelled as it
 * runs: the task list is cut into contiguous ranges, one per XCD, by the kernel's xcdTask rule
 * (equal task counts unless an XCD would get more than 3% above the mean panel count, then equal
 * panel counts with each boundary clamped to a quarter share from its equal-count place);
 * an XCD keeps `waves` tasks resident, gives them one panel each in turn, and starts the next task of
 * its range in a slot whose task has finished, the last 512 tasks of the range longest size class
 * first. One panel touches, in order:
 *   its sourceIds line, its sourceMetadata line, the values lines of its value range (A stream);
 *   then per slot (padding slots excluded) the F/128 lines of the source's packed X row and the
 *   line of its 4-byte scale.
 * Y and the partial tiles are written once by nontemporal or plain stores and are not replayed; the
 * caller adds their bytes.
 *
 * Policies: 0 LRU (what the hardware approximates), 1 optimal replacement (Belady: on a miss with the
 * set full, evict the line whose next use is furthest, or do not allocate the new line when its own
 * next use is furthest), 2 unbounded capacity (every distinct line misses once: the cold misses).
 * Policy 1 gives the fewest misses any replacement policy could reach on this access order and
 * capacity.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { S_X = 0, S_SCALE = 1, S_IDS = 2, S_META = 3, S_VALUES = 4, NSTREAMS = 5 };

typedef struct {
    uint32_t taskCount;
    const uint32_t* tasks;      /* Sw32Task[taskCount] as 7 u32 each: sw, begin, end, ... */
    const uint32_t* sourceIds;  /* 8 per panel, UINT32_MAX = padding */
    const uint32_t* panelBase;  /* value base of each panel's first slot (metadata >> 32) */
    uint64_t panels, values;    /* panel and value counts */
    uint32_t cols, features;
    uint32_t xcds, xcd;         /* model XCD `xcd` of `xcds` */
    uint32_t waves;             /* resident tasks per XCD */
    uint32_t lines, ways;       /* L2 capacity in 128-byte lines, associativity */
    uint32_t policy;            /* 0 LRU, 1 optimal, 2 unbounded */
    uint32_t bypassStreams;     /* bit s: accesses of stream s never allocate a line (hit if present) */
    uint32_t farRows;           /* > 0: X and scale accesses of sources farther than this many rows */
    uint32_t farStreams;        /*      from the SW's rows bypass too, for the streams in this mask  */
} l2m_input;

typedef struct {
    uint64_t accesses[NSTREAMS];
    uint64_t misses[NSTREAMS];
} l2m_result;

/* ---- access sequence of one XCD --------------------------------------------------------------- */

typedef struct {
    uint32_t* key;  /* line id, streams laid out one after another */
    uint8_t* stream;
    uint64_t n, cap;
} seq_t;

static int seq_push(seq_t* s, uint32_t key, uint8_t stream) {
    if (s->n == s->cap) {
        uint64_t cap = s->cap ? s->cap * 2 : (1u << 20);
        uint32_t* k = (uint32_t*)realloc(s->key, cap * sizeof(uint32_t));
        if (!k) return -1;
        s->key = k;
        uint8_t* t = (uint8_t*)realloc(s->stream, cap);
        if (!t) return -1;
        s->stream = t;
        s->cap = cap;
    }
    s->key[s->n] = key;
    s->stream[s->n] = stream;
    ++s->n;
    return 0;
}

typedef struct {
    uint64_t xBase, scaleBase, idsBase, metaBase, valuesBase, total;
} layout_t;

static layout_t make_layout(const l2m_input* in) {
    layout_t L;
    const uint64_t slots = in->panels * 8;
    L.xBase = 0;
    L.scaleBase = L.xBase + (uint64_t)in->cols * (in->features / 128);
    L.idsBase = L.scaleBase + ((uint64_t)in->cols * 4 + 127) / 128;
    L.metaBase = L.idsBase + (slots * 4 + 127) / 128;
    L.valuesBase = L.metaBase + (slots * 8 + 127) / 128;
    L.total = L.valuesBase + (in->values * 4 + 127) / 128;
    return L;
}

#define BYPASS 0x80u

static int panel_accesses(const l2m_input* in, const layout_t* L, uint64_t p, uint32_t sw, seq_t* s) {
    if (seq_push(s, (uint32_t)(L->idsBase + p * 32 / 128), S_IDS)) return -1;
    if (seq_push(s, (uint32_t)(L->metaBase + p * 64 / 128), S_META)) return -1;
    const uint64_t v0 = in->panelBase[p];
    const uint64_t v1 = p + 1 < in->panels ? in->panelBase[p + 1] : in->values;
    for (uint64_t l = v0 * 4 / 128; v1 > v0 && l <= (v1 * 4 - 1) / 128; ++l)
        if (seq_push(s, (uint32_t)(L->valuesBase + l), S_VALUES)) return -1;
    const uint32_t slices = in->features / 128;
    for (int k = 0; k < 8; ++k) {
        const uint32_t src = in->sourceIds[p * 8 + k];
        if (src == 0xFFFFFFFFu || src >= in->cols) continue;
        const int64_t row0 = (int64_t)sw * 32, d = (int64_t)src < row0 ? row0 - src : (int64_t)src - row0 - 31;
        const int far = in->farRows && d > (int64_t)in->farRows;
        const uint8_t fx = (far && (in->farStreams >> S_X & 1u)) ? BYPASS : 0;
        const uint8_t fs = (far && (in->farStreams >> S_SCALE & 1u)) ? BYPASS : 0;
        for (uint32_t j = 0; j < slices; ++j)
            if (seq_push(s, (uint32_t)(L->xBase + (uint64_t)src * slices + j), S_X | fx)) return -1;
        if (seq_push(s, (uint32_t)(L->scaleBase + src / 32), S_SCALE | fs)) return -1;
    }
    return 0;
}

/* The XCD's task range in the kernel's dispatch order: list order, except that the last TAIL_WINDOW
 * tasks of the range run longest size class first (panel counts >= 288, >= 192, >= 96, the rest;
 * list order within a class). */
enum { TAIL_WINDOW = 512 };

typedef struct {
    const l2m_input* in;
    uint32_t next, hi, w0;
    uint32_t window[TAIL_WINDOW];
} task_queue_t;

static uint32_t size_class(const l2m_input* in, uint32_t t) {
    const uint32_t* r = in->tasks + (uint64_t)t * 7;
    const uint32_t p = r[2] - r[1];
    return (uint32_t)(p >= 96) + (uint32_t)(p >= 192) + (uint32_t)(p >= 288);
}

static void queue_init(task_queue_t* tq, const l2m_input* in, uint32_t lo, uint32_t hi) {
    const uint32_t n = hi - lo < TAIL_WINDOW ? hi - lo : TAIL_WINDOW;
    tq->in = in;
    tq->next = lo;
    tq->hi = hi;
    tq->w0 = hi - n;
    uint32_t k = 0;
    for (int c = 3; c >= 0; --c)
        for (uint32_t t = tq->w0; t < hi; ++t)
            if (size_class(in, t) == (uint32_t)c) tq->window[k++] = t;
}

/* Gives slot w the next task with at least one panel; returns 0 when the range is exhausted. */
static int take_task(task_queue_t* tq, uint64_t* pos, uint64_t* end, uint32_t* sw) {
    while (tq->next < tq->hi) {
        const uint32_t i = tq->next++;
        const uint32_t task = i >= tq->w0 ? tq->window[i - tq->w0] : i;
        const uint32_t* t = tq->in->tasks + (uint64_t)task * 7;
        if (t[2] > t[1]) {
            *pos = t[1];
            *end = t[2];
            *sw = t[0];
            return 1;
        }
    }
    *pos = *end = 0;
    return 0;
}

/* Boundary k of the XCD ranges (xcdTask in spmm.hip, for any XCD count): equal task counts, or,
 * when that leaves an XCD more than 3% above the mean panel count, the first task starting at or
 * past k/xcds of the panels, clamped to half the spare share (ceil(T / (2 xcds)) workgroups per XCD)
 * from its equal-count place. */
static uint32_t equal_bound(uint32_t count, uint32_t xcds, uint32_t k) {
    const uint32_t q = count / xcds, r = count % xcds;
    return k * q + (k < r ? k : r);
}

static uint32_t task_begin(const l2m_input* in, uint32_t t) {
    return t < in->taskCount ? in->tasks[(uint64_t)t * 7 + 1] : in->tasks[(uint64_t)(in->taskCount - 1) * 7 + 2];
}

static uint32_t xcd_bound(const l2m_input* in, uint32_t k) {
    const uint32_t count = in->taskCount, xcds = in->xcds;
    if (k == 0 || k >= xcds || count == 0) return equal_bound(count, xcds, k);
    const uint64_t panels = task_begin(in, count);
    uint64_t maxPanels = 0;
    for (uint32_t j = 0; j < xcds; ++j) {
        const uint64_t n = task_begin(in, equal_bound(count, xcds, j + 1)) - task_begin(in, equal_bound(count, xcds, j));
        if (n > maxPanels) maxPanels = n;
    }
    const uint32_t eq = equal_bound(count, xcds, k);
    if (maxPanels * xcds * 100 <= panels * 103) return eq;
    const uint32_t target = (uint32_t)(panels * k / xcds);
    uint32_t lo = 0, hi = count;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (task_begin(in, mid) < target) lo = mid + 1;
        else hi = mid;
    }
    const uint32_t reach = ((count + 2 * xcds - 1) / (2 * xcds)) / 2;
    const uint32_t floorB = eq > reach ? eq - reach : 0, ceilB = eq + reach;
    return lo < floorB ? floorB : (lo > ceilB ? ceilB : lo);
}

static int build_sequence(const l2m_input* in, const layout_t* L, seq_t* s) {
    task_queue_t tq;
    queue_init(&tq, in, xcd_bound(in, in->xcd), xcd_bound(in, in->xcd + 1));
    const uint32_t W = in->waves ? in->waves : 1;
    uint64_t* pos = (uint64_t*)calloc(W, sizeof(uint64_t));
    uint64_t* end = (uint64_t*)calloc(W, sizeof(uint64_t));
    uint32_t* sw = (uint32_t*)calloc(W, sizeof(uint32_t));
    if (!pos || !end || !sw) {
        free(pos);
        free(end);
        free(sw);
        return -1;
    }
    uint32_t active = 0;
    for (uint32_t w = 0; w < W; ++w) active += (uint32_t)take_task(&tq, &pos[w], &end[w], &sw[w]);
    int rc = 0;
    while (active && !rc) {
        for (uint32_t w = 0; w < W && !rc; ++w) {
            if (pos[w] == end[w]) continue; /* idle slot */
            rc = panel_accesses(in, L, pos[w]++, sw[w], s);
            if (pos[w] == end[w] && !take_task(&tq, &pos[w], &end[w], &sw[w])) --active;
        }
    }
    free(pos);
    free(end);
    free(sw);
    return rc;
}

/* ---- cache replay ------------------------------------------------------------------------------ */

static inline uint32_t set_of(uint32_t key, uint32_t sets) {
    uint64_t h = (uint64_t)key * 0x9E3779B97F4A7C15ull;
    return (uint32_t)((h >> 32) % sets);
}

static int replay(const l2m_input* in, const seq_t* s, uint64_t keyspace, l2m_result* out) {
    const uint64_t n = s->n;
    if (in->policy == 2) {
        uint8_t* seen = (uint8_t*)calloc(keyspace, 1);
        if (!seen) return -1;
        for (uint64_t i = 0; i < n; ++i) {
            const unsigned st = s->stream[i] & 0x7Fu;
            out->accesses[st]++;
            if (!seen[s->key[i]]) {
                seen[s->key[i]] = 1;
                out->misses[st]++;
            }
        }
        free(seen);
        return 0;
    }
    const uint32_t ways = in->ways, sets = in->lines / in->ways;
    uint32_t* tag = (uint32_t*)malloc((uint64_t)sets * ways * sizeof(uint32_t));
    uint64_t* stamp = (uint64_t*)malloc((uint64_t)sets * ways * sizeof(uint64_t));
    uint32_t* nextUse = NULL;
    if (!tag || !stamp) return -1;
    memset(tag, 0xFF, (uint64_t)sets * ways * sizeof(uint32_t));
    memset(stamp, 0, (uint64_t)sets * ways * sizeof(uint64_t));
    if (in->policy == 1) { /* next use of each access, by a backward scan */
        nextUse = (uint32_t*)malloc(n * sizeof(uint32_t));
        uint32_t* last = (uint32_t*)malloc(keyspace * sizeof(uint32_t));
        if (!nextUse || !last) return -1;
        memset(last, 0xFF, keyspace * sizeof(uint32_t));
        for (uint64_t i = n; i-- > 0;) {
            nextUse[i] = last[s->key[i]];
            last[s->key[i]] = (uint32_t)i;
        }
        free(last);
    }
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t key = s->key[i];
        const unsigned st = s->stream[i] & 0x7Fu;
        const int bypass = (s->stream[i] & BYPASS) || (in->bypassStreams >> st & 1u);
        out->accesses[st]++;
        const uint64_t base = (uint64_t)set_of(key, sets) * ways;
        int hit = -1, empty = -1;
        for (uint32_t w = 0; w < ways; ++w) {
            if (tag[base + w] == key) hit = (int)w;
            else if (tag[base + w] == 0xFFFFFFFFu && empty < 0) empty = (int)w;
        }
        /* stamp: LRU = time of last use; optimal = time of next use (UINT32_MAX = never) */
        const uint64_t mark = in->policy == 1 ? (uint64_t)nextUse[i] : i + 1;
        if (hit >= 0) {
            stamp[base + hit] = mark;
            continue;
        }
        out->misses[st]++;
        if (bypass) continue;
        if (empty >= 0) {
            tag[base + empty] = key;
            stamp[base + empty] = mark;
            continue;
        }
        uint32_t victim = 0;
        for (uint32_t w = 1; w < ways; ++w) {
            const int better = in->policy == 1 ? stamp[base + w] > stamp[base + victim]
                                               : stamp[base + w] < stamp[base + victim];
            if (better) victim = w;
        }
        if (in->policy == 1 && mark >= stamp[base + victim]) continue; /* bypass */
        tag[base + victim] = key;
        stamp[base + victim] = mark;
    }
    free(tag);
    free(stamp);
    free(nextUse);
    return 0;
}

/* Returns 0 on success, -1 on allocation failure, -2 on invalid input. */
int l2m_replay(const l2m_input* in, l2m_result* out) {
    memset(out, 0, sizeof(*out));
    if (!in || !in->xcds || in->xcd >= in->xcds || !in->features || in->features % 128 ||
        (in->policy != 2 && (!in->ways || !in->lines || in->lines % in->ways)))
        return -2;
    const layout_t L = make_layout(in);
    if (L.total >= 0xFFFFFFFFull) return -2;
    seq_t s = {0};
    int rc = build_sequence(in, &L, &s);
    if (!rc) rc = replay(in, &s, L.total, out);
    free(s.key);
    free(s.stream);
    return rc;
}
