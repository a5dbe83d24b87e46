/* Canonical sequential semantics of the device expert cache and the host RAM-tier admission step.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP ensure kernel and the product's host step, never linked into the
 * product.
 *
 * Restates (paths relative to the reference repository root):
 *   kernels/moe-a8/exl3_moe.a8.sycl:864-1039   launch_ensure, decode mode, with work-items taken in index order:
 *                                              tier mask + miss ring (902-914), need set (915), hits/misses (917-923),
 *                                              exact-LRU victims by the nm-th smallest u = slot_last + 1 among slots not
 *                                              touched this tick (929-1000), assignment + old-owner repoint (1003-1023)
 *   kernels/moe-a8/exl3_moe.a8.sycl:1168-1189  VictimCopyKernel: ram_res[old] = 1 for written-back victims
 *   kernels/moe-a8/exl3_moe.a8.sycl:846-851, 884, 1019-1021, 1194-1222
 *                                              prefetch mode (moe_prefetch): the tick is not advanced (slots of the last
 *                                              call, last == T, stay protected), no tier mask, no write-back, the
 *                                              assigned slots are the pf_slot list
 *   kernels/moe-a8/exl3_moe.a8.sycl:853-901, 1013-1038, 1127-1142
 *                                              copy-engine plan mode (moe_prefetch_plan): prefetch mode with at most 16
 *                                              misses, claimed slots pinned (slot_last = INT_MAX) and recorded as the
 *                                              layer's pending plan; a layer with a pending plan is skipped; every call
 *                                              first commits the finished pending plans (slot_last = the plan's tick).
 *                                              Here a plan is finished by the next call (the caller waits for the copy
 *                                              worker), the protocol the tests follow.
 *   plugin/exl3xpu/nvtier.py:57-87, 179-188    tier init (pinned safe expert per layer, tick = 1)
 *   plugin/exl3xpu/nvtier.py:282-386, 708-806  NvTierAsync one-step-lagged snapshot + _async_step_admit
 *   experimental/n111-victim-ring/a9.patch:46-65, nvtier.py:655-884
 *                                              victim ring (co_set_ring): the ensure claims ring slots for written-back
 *                                              victims serially in victim order (free slot = key < 0, searched
 *                                              circularly from the next search position; none free: dropped), never
 *                                              flags them RAM-resident; the host step takes the new claims of the
 *                                              lagged snapshot into flight and lands them one host step later (RAM-
 *                                              resident like a completed fill, the slot freed before the next call)
 *
 * Canonical choices where the reference is not deterministic (documented contract):
 *   - misses in ascending expert id; victims = ascending-slot({u < tau}) ++ first `want` of ascending-slot({u == tau});
 *   - ring entries in ascending pick index;
 *   - host age ties broken by ascending key (stable sort), the reference uses numpy's default unstable argsort;
 *   - NVMe completions: a fill admitted at host step n completes at host step n + latency.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int L, E, S, R, tier;
    int budget, age_min, qmax, latency;
    /* device state */
    int32_t *slot_of, *slot_key, *slot_last, tick;
    uint8_t *ram_res;
    int32_t *ring;           /* [1 + R] */
    int32_t *safe;           /* [L] */
    /* host state */
    uint8_t *res, *inflight, *pin;
    int64_t *age, htick, ring_seen;
    int k;                   /* snapshot toggle */
    int have_snap[2];
    uint8_t *snap_res[2];
    int32_t *snap_ring[2];
    uint8_t *snap_vram[2];
    int32_t *last_dk; uint8_t *last_dv; int64_t n_last;
    int32_t **done; int64_t *n_done;   /* [latency + 1] ring of completion lists */
    int64_t hstep;
    /* scratch */
    uint32_t *u_tmp; int32_t *i_tmp; int64_t *l_tmp, *l_tmp2; int32_t *cnt_tmp; uint8_t *view, *resn;
    int64_t stats_masked, stats_evicts, stats_admit_dropped, stats_ring_overflow;
    /* pending copy-engine prefetch plans per layer: count, tick, (expert, slot) x 16 */
    int32_t *pend_n, *pend_T, *pend_e, *pend_s;
    /* victim ring (vr_K = 0: off): device meta, its snapshots, the host's handled claim numbers, the claims taken
     * into flight by the last host step (they land at the next one) and the slots to free */
    int vr_K, vr_p, vr_claims, vr_drops, vr_error;
    int32_t *vr_key, *vr_seq, *snap_vr[2];
    int64_t *vr_seen;
    int32_t *vr_fly_r, *vr_fly_k, vr_n_fly, *vr_free, vr_n_free;
} co_t;

static void *xcalloc(size_t n, size_t s) { void *p = calloc(n ? n : 1, s); return p; }

co_t *co_new(int L, int E, int S, int ring_cap, int tier, int budget, int age_min, int qmax, int latency, int safe) {
    co_t *c = (co_t *)xcalloc(1, sizeof(co_t));
    int n = L * E;
    c->L = L; c->E = E; c->S = S; c->R = ring_cap; c->tier = tier;
    c->budget = budget; c->age_min = age_min; c->qmax = qmax; c->latency = latency;
    c->slot_of = (int32_t *)xcalloc(n, 4); c->slot_key = (int32_t *)xcalloc(S, 4); c->slot_last = (int32_t *)xcalloc(S, 4);
    for (int i = 0; i < n; ++i) c->slot_of[i] = -1;
    for (int s = 0; s < S; ++s) { c->slot_key[s] = -1; c->slot_last[s] = -1; }
    c->ram_res = (uint8_t *)xcalloc(n, 1);
    c->ring = (int32_t *)xcalloc(1 + ring_cap, 4);
    c->safe = (int32_t *)xcalloc(L, 4);
    c->res = (uint8_t *)xcalloc(n, 1); c->inflight = (uint8_t *)xcalloc(n, 1); c->pin = (uint8_t *)xcalloc(n, 1);
    c->age = (int64_t *)xcalloc(n, 8);
    c->htick = 1;
    for (int li = 0; li < L; ++li) {
        c->safe[li] = safe;
        if (tier) { c->res[li * E + safe] = 1; c->pin[li * E + safe] = 1; c->ram_res[li * E + safe] = 1; }
    }
    for (int b = 0; b < 2; ++b) {
        c->snap_res[b] = (uint8_t *)xcalloc(n, 1); c->snap_ring[b] = (int32_t *)xcalloc(1 + ring_cap, 4);
        c->snap_vram[b] = (uint8_t *)xcalloc(n, 1);
    }
    c->last_dk = (int32_t *)xcalloc(n, 4); c->last_dv = (uint8_t *)xcalloc(n, 1);
    c->done = (int32_t **)xcalloc(latency + 1, sizeof(int32_t *));
    c->n_done = (int64_t *)xcalloc(latency + 1, 8);
    for (int i = 0; i <= latency; ++i) c->done[i] = (int32_t *)xcalloc(qmax > 0 ? qmax : 1, 4);
    c->u_tmp = (uint32_t *)xcalloc(S, 4); c->i_tmp = (int32_t *)xcalloc(S > E ? S : E, 4);
    c->l_tmp = (int64_t *)xcalloc(n > ring_cap ? n : ring_cap, 8); c->l_tmp2 = (int64_t *)xcalloc(n > ring_cap ? n : ring_cap, 8);
    c->cnt_tmp = (int32_t *)xcalloc(n, 4);
    c->view = (uint8_t *)xcalloc(n, 1); c->resn = (uint8_t *)xcalloc(n, 1);
    c->pend_n = (int32_t *)xcalloc(L, 4); c->pend_T = (int32_t *)xcalloc(L, 4);
    c->pend_e = (int32_t *)xcalloc((size_t)L * 16, 4); c->pend_s = (int32_t *)xcalloc((size_t)L * 16, 4);
    return c;
}

void co_free(co_t *c) {
    if (!c) return;
    free(c->slot_of); free(c->slot_key); free(c->slot_last); free(c->ram_res); free(c->ring); free(c->safe);
    free(c->res); free(c->inflight); free(c->pin); free(c->age);
    for (int b = 0; b < 2; ++b) { free(c->snap_res[b]); free(c->snap_ring[b]); free(c->snap_vram[b]); }
    free(c->last_dk); free(c->last_dv);
    for (int i = 0; i <= c->latency; ++i) free(c->done[i]);
    free(c->done); free(c->n_done);
    free(c->u_tmp); free(c->i_tmp); free(c->l_tmp); free(c->l_tmp2); free(c->cnt_tmp); free(c->view); free(c->resn);
    free(c->pend_n); free(c->pend_T); free(c->pend_e); free(c->pend_s);
    if (c->vr_K) {
        free(c->vr_key); free(c->vr_seq); free(c->snap_vr[0]); free(c->snap_vr[1]); free(c->vr_seen);
        free(c->vr_fly_r); free(c->vr_fly_k); free(c->vr_free);
    }
    free(c);
}

/* turn the victim ring on with K slots (before the first call) */
void co_set_ring(co_t *c, int K) {
    c->vr_K = K; c->vr_p = 0; c->vr_claims = 0; c->vr_drops = 0; c->vr_error = 0;
    c->vr_key = (int32_t *)xcalloc(K, 4); c->vr_seq = (int32_t *)xcalloc(K, 4);
    for (int r = 0; r < K; ++r) c->vr_key[r] = -1;
    for (int b = 0; b < 2; ++b) {
        c->snap_vr[b] = (int32_t *)xcalloc(2 * (size_t)K, 4);
        for (int r = 0; r < K; ++r) c->snap_vr[b][r] = -1;
    }
    c->vr_seen = (int64_t *)xcalloc(K, 8);
    c->vr_fly_r = (int32_t *)xcalloc(K, 4); c->vr_fly_k = (int32_t *)xcalloc(K, 4); c->vr_n_fly = 0;
    c->vr_free = (int32_t *)xcalloc(2 * (size_t)K, 4); c->vr_n_free = 0;
}
int32_t *co_vr_key(co_t *c) { return c->vr_key; }
int32_t *co_vr_seq(co_t *c) { return c->vr_seq; }
void co_vr_stats(co_t *c, int64_t *out) {
    out[0] = c->vr_p; out[1] = c->vr_claims; out[2] = c->vr_drops; out[3] = c->vr_error;
}

/* state accessors (ctypes maps them onto numpy arrays) */
int32_t *co_slot_of(co_t *c) { return c->slot_of; }
int32_t *co_slot_key(co_t *c) { return c->slot_key; }
int32_t *co_slot_last(co_t *c) { return c->slot_last; }
int32_t *co_tick(co_t *c) { return &c->tick; }
uint8_t *co_ram_res(co_t *c) { return c->ram_res; }
int32_t *co_ring(co_t *c) { return c->ring; }
int32_t *co_safe(co_t *c) { return c->safe; }
uint8_t *co_res(co_t *c) { return c->res; }
uint8_t *co_inflight(co_t *c) { return c->inflight; }
int64_t *co_age(co_t *c) { return c->age; }
int64_t co_htick(co_t *c) { return c->htick; }
void co_stats(co_t *c, int64_t *out) {
    out[0] = c->stats_masked; out[1] = c->stats_evicts; out[2] = c->stats_admit_dropped; out[3] = c->stats_ring_overflow;
}

/* quickselect: k-th smallest (0-based) of a[0..n) (a is modified) */
static uint32_t kth_smallest(uint32_t *a, int n, int k) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        uint32_t p = a[lo + (hi - lo) / 2];
        int i = lo, j = hi;
        while (i <= j) {
            while (a[i] < p) ++i;
            while (a[j] > p) --j;
            if (i <= j) { uint32_t t = a[i]; a[i] = a[j]; a[j] = t; ++i; --j; }
        }
        if (k <= j) hi = j;
        else if (k >= i) lo = i;
        else return a[k];
    }
    return a[k];
}

/* Record layout per ensure call, P = number of picks (int32):
 *   [0] T   [1] ring count after the call   [2, 2+P) post-mask ids   [2+P] nm
 *   [3+P, 3+2P) assigned miss experts (fill_list order, -1 pad)   [3+2P, 3+4P) (old-or-minus-1, slot) pairs (-2 pad)
 */
int co_rec_len(int P) { return 3 + 4 * P; }

/* mode: 0 decode, 1 prefetch, 2 copy-engine plan */
static int ensure_impl(co_t *c, int layer, int32_t *ids, float *w, int P, int max_fill, int32_t *rec, int mode) {
    const int E = c->E, S = c->S;
    const int prefetch = mode != 0, plan = mode == 2;
    for (int li = 0; li < c->L && mode != 1; ++li) {           /* commit finished plans (a8:856-880; not in a
                                                                  * prefetch call, which has no pending table) */
        for (int i = 0; i < c->pend_n[li]; ++i) c->slot_last[c->pend_s[li * 16 + i]] = c->pend_T[li];
        c->pend_n[li] = 0;
    }
    const int32_t T = prefetch ? c->tick : ++c->tick;          /* a8:884 */
    const int tier = c->tier && !prefetch;                     /* prefetch: no mask, no write-back (a8:846-851) */
    int32_t *need = c->cnt_tmp;                                /* E entries used */
    int32_t *miss = c->i_tmp;
    if (tier) {                                                /* a8:902-914 */
        for (int i = 0; i < P; ++i) {
            int key = layer * E + ids[i];
            if (c->slot_of[key] < 0 && !c->ram_res[key]) {
                uint32_t cnt = (uint32_t)c->ring[0];          /* the count wraps modulo 2^32 */
                c->ring[0] = (int32_t)(cnt + 1u);
                c->ring[1 + (int)(cnt % (uint32_t)c->R)] = key;
                ids[i] = c->safe[layer];
                w[i] = 0.0f;
                c->stats_masked++;
            }
        }
    }
    for (int e = 0; e < E; ++e) need[e] = 0;
    for (int i = 0; i < P; ++i) need[ids[i]] = 1;              /* a8:915 */
    int nmiss = 0;
    for (int e = 0; e < E; ++e) {                              /* a8:917-923 */
        if (!need[e]) continue;
        int s = c->slot_of[layer * E + e];
        if (s >= 0) { if (c->slot_last[s] != 0x7FFFFFFF) c->slot_last[s] = T; }
        else miss[nmiss++] = e;
    }
    int mf = max_fill < E ? max_fill : E;
    if (plan && mf > 16) mf = 16;                              /* a8:1135 */
    int nm = S > 0 ? (nmiss < mf ? nmiss : mf) : 0;
    int nelig = 0;
    if (nm > 0) {
        for (int s = 0; s < S; ++s) if (c->slot_last[s] < T) c->u_tmp[nelig++] = (uint32_t)(c->slot_last[s] + 1);
        if (nm > nelig) nm = nelig;
    }
    if (rec) {
        rec[0] = T;
        for (int i = 0; i < P; ++i) rec[2 + i] = ids[i];
        for (int i = 0; i < P; ++i) rec[3 + P + i] = -1;
        for (int i = 0; i < 2 * P; ++i) rec[3 + 2 * P + i] = -2;
    }
    if (nm > 0) {
        uint32_t tau = kth_smallest(c->u_tmp, nelig, nm - 1);  /* nm-th smallest u, with multiplicity */
        int n_lt = 0;
        for (int s = 0; s < S; ++s) if (c->slot_last[s] < T && (uint32_t)(c->slot_last[s] + 1) < tau) ++n_lt;
        int want = nm - n_lt;
        int32_t *V = (int32_t *)malloc(sizeof(int32_t) * nm);
        int iv = 0, ieq = 0;
        for (int s = 0; s < S; ++s)
            if (c->slot_last[s] < T && (uint32_t)(c->slot_last[s] + 1) < tau) V[iv++] = s;
        for (int s = 0; s < S && ieq < want; ++s)
            if (c->slot_last[s] < T && (uint32_t)(c->slot_last[s] + 1) == tau) { V[iv++] = s; ++ieq; }
        for (int mi = 0; mi < nm; ++mi) {                      /* a8:1003-1023 */
            int s = V[mi], e = miss[mi];
            int old = c->slot_key[s];
            int wb = old;
            if (tier && old >= 0 && c->ram_res[old]) wb = -1;
            if (old >= 0) c->slot_of[old] = -1;
            int key = layer * E + e;
            c->slot_key[s] = key; c->slot_of[key] = s; c->slot_last[s] = plan ? 0x7FFFFFFF : T;
            if (plan) { c->pend_e[layer * 16 + mi] = e; c->pend_s[layer * 16 + mi] = s; }
            if (tier && wb >= 0 && c->vr_K) {                  /* ring claim, a9.patch:50-63 */
                int r = -1;
                for (int j = 0; j < c->vr_K; ++j) {
                    int q = c->vr_p + j;
                    if (q >= c->vr_K) q -= c->vr_K;
                    if (c->vr_key[q] < 0) { r = q; break; }
                }
                if (r >= 0) {
                    c->vr_key[r] = wb; c->vr_seq[r] = ++c->vr_claims;
                    c->vr_p = r + 1 == c->vr_K ? 0 : r + 1;
                } else {
                    c->vr_drops += 1;
                    wb = -1;                                    /* dropped: no write-back */
                }
            }
            if (rec) { rec[3 + P + mi] = e; rec[3 + 2 * P + 2 * mi] = wb; rec[3 + 2 * P + 2 * mi + 1] = s; }
            if (tier && wb >= 0 && !c->vr_K) c->ram_res[wb] = 1;   /* VictimCopyKernel a8:1180 */
        }
        free(V);
    }
    if (plan && nm > 0) { c->pend_n[layer] = nm; c->pend_T[layer] = T; }
    if (rec) { rec[1] = c->ring[0]; rec[2 + P] = nm; }
    return nm;
}

int co_ensure(co_t *c, int layer, int32_t *ids, float *w, int P, int max_fill, int32_t *rec) {
    return ensure_impl(c, layer, ids, w, P, max_fill, rec, 0);
}

/* moe_prefetch's ensure (a8:1194-1222): same record layout; the assigned (expert, slot) pairs are the fill_list /
 * pf_slot lists, and the old owner's record field holds the old key (no write-back decision) */
int co_prefetch(co_t *c, int layer, int32_t *ids, int P, int max_fill, int32_t *rec) {
    return ensure_impl(c, layer, ids, NULL, P, max_fill, rec, 1);
}

/* moe_prefetch_plan's ensure (a8:1127-1142): a prefetch whose claimed slots stay pinned until the next call */
int co_plan(co_t *c, int layer, int32_t *ids, int P, int max_fill, int32_t *rec) {
    return ensure_impl(c, layer, ids, NULL, P, max_fill, rec, 2);
}

/* stable sort of keys[0..n) by age ascending (ties: keys are already ascending) */
static int64_t *g_age_for_sort;
static int cmp_age(const void *a, const void *b) {
    int64_t ka = *(const int64_t *)a, kb = *(const int64_t *)b;
    int64_t aa = g_age_for_sort[ka], ab = g_age_for_sort[kb];
    if (aa != ab) return aa < ab ? -1 : 1;
    return ka < kb ? -1 : (ka > kb);
}
static int32_t *g_cnt_for_sort;
static int cmp_cnt_desc(const void *a, const void *b) {
    int64_t ka = *(const int64_t *)a, kb = *(const int64_t *)b;
    int32_t ca = g_cnt_for_sort[ka], cb = g_cnt_for_sort[kb];
    if (ca != cb) return ca > cb ? -1 : 1;
    return ka < kb ? -1 : (ka > kb);
}
static int cmp_i64(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return x < y ? -1 : (x > y);
}

/* Host step n (after device step n). Writes admitted and evicted keys; returns the number of new ring entries
 * consumed (0 on the first call). The device flag upload (diff) is applied to ram_res at the end. */
int64_t co_host_step(co_t *c, int32_t *admit_out, int32_t *n_admit, int32_t *evict_out, int32_t *n_evict) {
    const int n = c->L * c->E;
    *n_admit = 0; *n_evict = 0;
    c->htick += 1;
    int k = c->k; c->k ^= 1;
    memcpy(c->snap_res[k], c->ram_res, n);
    memcpy(c->snap_ring[k], c->ring, 4 * (size_t)(1 + c->R));
    for (int i = 0; i < n; ++i) c->snap_vram[k][i] = c->slot_of[i] >= 0;
    if (c->vr_K) {
        memcpy(c->snap_vr[k], c->vr_key, 4 * (size_t)c->vr_K);
        memcpy(c->snap_vr[k] + c->vr_K, c->vr_seq, 4 * (size_t)c->vr_K);
    }
    c->have_snap[k] = 1;
    int j = k ^ 1;
    int64_t hstep = c->hstep++;
    int slot_now = (int)(hstep % (c->latency + 1));
    if (!c->have_snap[j]) return 0;
    uint8_t *view = c->view, *res = c->resn;
    memcpy(view, c->snap_res[j], n);
    for (int64_t i = 0; i < c->n_last; ++i) view[c->last_dk[i]] = c->last_dv[i];
    const int32_t *ring = c->snap_ring[j];
    const uint8_t *vram = c->snap_vram[j];
    memcpy(res, c->res, n);
    for (int i = 0; i < n; ++i)
        if (view[i] == 1 && c->res[i] == 0) { c->age[i] = c->htick; res[i] = 1; }   /* nvtier.py:757-761 */
    for (int64_t i = 0; i < c->n_done[slot_now]; ++i) {                           /* nvtier.py:762-763 */
        int kk = c->done[slot_now][i];
        res[kk] = 1; c->age[kk] = c->htick; c->inflight[kk] = 0;
    }
    c->n_done[slot_now] = 0;
    if (c->vr_K) {
        /* ring drains taken into flight by the last host step land now (n111 nvtier.py:787-794) */
        for (int i = 0; i < c->vr_n_fly; ++i) {
            int kk = c->vr_fly_k[i];
            res[kk] = 1; c->age[kk] = c->htick; c->inflight[kk] = 0;
            c->vr_free[c->vr_n_free++] = c->vr_fly_r[i];
        }
        c->vr_n_fly = 0;
        /* new claims of the snapshot (n111 nvtier.py:798-806): in flight, or, when the key is RAM-resident already,
         * nothing to copy and the slot is freed */
        const int32_t *sk = c->snap_vr[j], *ss = c->snap_vr[j] + c->vr_K;
        for (int r = 0; r < c->vr_K; ++r) {
            if (sk[r] < 0 || ss[r] == c->vr_seen[r]) continue;
            c->vr_seen[r] = ss[r];
            int kk = sk[r];
            if (c->res[kk]) { c->vr_free[c->vr_n_free++] = r; continue; }
            if (c->inflight[kk]) c->vr_error = 1;
            c->inflight[kk] = 1;
            c->vr_fly_r[c->vr_n_fly] = r; c->vr_fly_k[c->vr_n_fly++] = kk;
        }
    }
    /* new misses with multiplicity (nvtier.py:765-775) */
    /* the device count wraps modulo 2^32 (the reference's Python int does not; it never reaches 2^31 in its runs) */
    uint32_t cnt = (uint32_t)ring[0];
    int64_t newm = (int64_t)(uint32_t)(cnt - (uint32_t)c->ring_seen), cap = c->R;
    if (newm > cap) { c->stats_ring_overflow += newm - cap; newm = cap; }
    int64_t nwant = 0;
    int64_t *want = c->l_tmp;
    if (newm > 0) {
        int64_t *keys = c->l_tmp2;
        for (int64_t i = 0; i < newm; ++i) {
            int64_t pos = (int64_t)((uint32_t)(cnt - (uint32_t)(newm - i)) % (uint32_t)cap);
            keys[i] = ring[1 + pos];
        }
        qsort(keys, (size_t)newm, 8, cmp_i64);
        int64_t nu = 0;
        for (int64_t i = 0; i < newm; ++i) {
            if (nu == 0 || keys[nu - 1] != keys[i]) { keys[nu] = keys[i]; c->cnt_tmp[keys[i]] = 1; ++nu; }
            else c->cnt_tmp[keys[i]] += 1;
        }
        for (int64_t i = 0; i < nu; ++i)
            if (res[keys[i]] == 0 && !c->inflight[keys[i]]) want[nwant++] = keys[i];
        g_cnt_for_sort = c->cnt_tmp;
        qsort(want, (size_t)nwant, 8, cmp_cnt_desc);
    }
    c->ring_seen = (int64_t)cnt;
    /* budget (nvtier.py:777-788) */
    int64_t inflight_n = 0, nres = 0;
    for (int i = 0; i < n; ++i) { inflight_n += c->inflight[i]; nres += res[i]; }
    int64_t over = nres + inflight_n + nwant - c->budget;
    if (over > 0) {
        int64_t *cand = (int64_t *)malloc(8 * (size_t)n);
        int64_t nc = 0;
        for (int i = 0; i < n; ++i) if (res[i] && vram[i] && !c->pin[i]) cand[nc++] = i;
        g_age_for_sort = c->age;
        qsort(cand, (size_t)nc, 8, cmp_age);
        int64_t t1 = nc < over ? nc : over;
        for (int64_t i = 0; i < t1; ++i) { evict_out[(*n_evict)++] = (int32_t)cand[i]; }
        over -= t1;
        if (over > 0) {
            nc = 0;
            for (int i = 0; i < n; ++i) if (res[i] && !c->pin[i] && c->age[i] <= c->htick - c->age_min) cand[nc++] = i;
            /* exclude take1 */
            int64_t m2 = 0;
            for (int64_t i = 0; i < nc; ++i) {
                int in1 = 0;
                for (int64_t q = 0; q < t1; ++q) if (evict_out[q] == cand[i]) { in1 = 1; break; }
                if (!in1) cand[m2++] = cand[i];
            }
            qsort(cand, (size_t)m2, 8, cmp_age);
            int64_t t2 = m2 < over ? m2 : over;
            for (int64_t i = 0; i < t2; ++i) evict_out[(*n_evict)++] = (int32_t)cand[i];
        }
        for (int i = 0; i < *n_evict; ++i) res[evict_out[i]] = 0;
        c->stats_evicts += *n_evict;
        free(cand);
    }
    nres = 0;
    for (int i = 0; i < n; ++i) nres += res[i];
    int64_t f1 = c->budget - nres - inflight_n, f2 = c->qmax - inflight_n;
    int64_t fr = f1 < f2 ? f1 : f2;
    if (fr < 0) fr = 0;
    int64_t nadm = nwant < fr ? nwant : fr;
    c->stats_admit_dropped += nwant - nadm;
    int slot_done = (int)((hstep + c->latency) % (c->latency + 1));
    for (int64_t i = 0; i < nadm; ++i) {
        int kk = (int)want[i];
        c->inflight[kk] = 1;
        admit_out[(*n_admit)++] = kk;
        c->done[slot_done][c->n_done[slot_done]++] = kk;
    }
    /* flag diff upload (nvtier.py:789-796) */
    c->n_last = 0;
    for (int i = 0; i < n; ++i)
        if (res[i] != view[i]) { c->last_dk[c->n_last] = i; c->last_dv[c->n_last] = res[i]; c->n_last++; c->ram_res[i] = res[i]; }
    memcpy(c->res, res, n);
    for (int i = 0; i < c->vr_n_free; ++i) c->vr_key[c->vr_free[i]] = -1;   /* before the next call */
    c->vr_n_free = 0;
    return newm > 0 ? newm : 0;
}

/* Drive a whole trace: ids/w [steps][L][P]; per call records [steps][L][rec_len]; per host step a log
 * [n_admit, n_evict, admits..., evicts...] appended to host_log (returns the number of int32 written, -1 if full). */
int64_t co_run(co_t *c, const int32_t *ids, const float *w, int steps, int P, int max_fill, int32_t *recs,
               int32_t *host_log, int64_t host_log_cap) {
    int rl = co_rec_len(P);
    int32_t *idb = (int32_t *)malloc(4 * (size_t)P);
    float *wb = (float *)malloc(4 * (size_t)P);
    int32_t *adm = (int32_t *)malloc(4 * (size_t)(c->qmax > 0 ? c->qmax : 1));
    int32_t *evc = (int32_t *)malloc(4 * (size_t)c->L * c->E);
    int64_t pos = 0;
    for (int n = 0; n < steps; ++n) {
        for (int li = 0; li < c->L; ++li) {
            size_t o = ((size_t)n * c->L + li) * P;
            memcpy(idb, ids + o, 4 * (size_t)P);
            memcpy(wb, w + o, 4 * (size_t)P);
            co_ensure(c, li, idb, wb, P, max_fill, recs ? recs + ((size_t)n * c->L + li) * rl : NULL);
        }
        if (c->tier) {
            int32_t na, ne;
            co_host_step(c, adm, &na, evc, &ne);
            if (host_log) {
                if (pos + 2 + na + ne > host_log_cap) { pos = -1; break; }
                host_log[pos++] = na; host_log[pos++] = ne;
                memcpy(host_log + pos, adm, 4 * (size_t)na); pos += na;
                memcpy(host_log + pos, evc, 4 * (size_t)ne); pos += ne;
            }
        }
    }
    free(idb); free(wb); free(adm); free(evc);
    return pos;
}
