// Host admission step of the RAM tier, native (the reference runs it as numpy: _async_step_admit,
// plugin/exl3xpu/nvtier.py:708-806, called from NvTierAsync.step nvtier.py:282-386).
//
// Stateless over caller-owned arrays: res / age / inflight are the host's books (updated in place), view is the
// device flag snapshot of the previous step with the previous upload overlaid, ring the device miss ring snapshot
// ([0] = monotonic count, then `ring_cap` keys), slot_of the HBM slot snapshot (>= 0 = resident in HBM).
//
// Decision order (each step's output is a pure function of these inputs):
//   1. flags the device set (victim write-back) become resident with age = tick;
//   2. fills completed now become resident with age = tick and leave the in-flight set;
//   3. keys missed since the last step, with multiplicity, that are neither resident nor in flight: `want`, by
//      descending miss count, ties by ascending key;
//   4. over budget (resident + in flight + wanted): evict first the RAM copies of HBM-resident keys, then keys older
//      than `admit_age` steps, each group by ascending age, ties by ascending key; pinned keys never;
//   5. admit the head of `want`, limited by the free budget and by `admit_qmax` fills in flight;
//   6. the flag diff to upload: every key whose books differ from the view.
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "../../include/exl3moe.h"

namespace {

struct Scratch {
    std::vector<int32_t> count;     // miss multiplicity per key (all zero between calls)
    std::vector<int64_t> touched, want, cand;
};
thread_local Scratch tls;

// the `k` candidates of smallest (age, key), written to out in that order
int64_t smallest_by_age(std::vector<int64_t>& cand, const int64_t* age, int64_t k, int64_t* out) {
    auto less = [age](int64_t a, int64_t b) { return age[a] != age[b] ? age[a] < age[b] : a < b; };
    k = std::min<int64_t>(k, (int64_t)cand.size());
    if (k <= 0) return 0;
    if (k < (int64_t)cand.size()) std::nth_element(cand.begin(), cand.begin() + k, cand.end(), less);
    std::sort(cand.begin(), cand.begin() + k, less);
    std::copy(cand.begin(), cand.begin() + k, out);
    return k;
}

}  // namespace

extern "C" int exl3_admit_decide(exl3_admit_state* st, uint8_t* res, int64_t* age, uint8_t* inflight,
                                 const uint8_t* pin, const uint8_t* view, const int32_t* ring, const int32_t* slot_of,
                                 const int64_t* done, int64_t n_done, int64_t* adm, int64_t* n_adm, int64_t* ev,
                                 int64_t* n_ev, int64_t* diff, uint8_t* vals, int64_t* n_diff) {
    if (!st || !res || !age || !inflight || !pin || !view || !ring || !slot_of || !adm || !n_adm || !ev || !n_ev ||
        !diff || !vals || !n_diff || (n_done > 0 && !done))
        return EXL3_EINVAL;
    const int64_t n = st->n, tick = st->tick, cap = st->ring_cap;
    if (n <= 0 || cap <= 0 || n_done < 0) return EXL3_EINVAL;
    for (int64_t i = 0; i < n_done; ++i)
        if (done[i] < 0 || done[i] >= n) return EXL3_EINVAL;
    if (cap > INT32_MAX) return EXL3_EINVAL;
    // the device ring count wraps modulo 2^32: the entries since the last step are (cnt - ring_seen) mod 2^32, and entry
    // c sits at position (c mod 2^32) % cap, the same formula the device uses when it writes
    const uint32_t cnt = (uint32_t)ring[0];
    int64_t newm = (int64_t)(uint32_t)(cnt - (uint32_t)st->ring_seen);
    const int64_t overflow = newm > cap ? newm - cap : 0;
    newm -= overflow;
    auto pos_of = [cnt, newm, cap](int64_t i) { return (int64_t)((uint32_t)(cnt - (uint32_t)(newm - i)) % (uint32_t)cap); };
    for (int64_t i = 0; i < newm; ++i) {         // validate before touching the books
        const int32_t key = ring[1 + pos_of(i)];
        if (key < 0 || key >= n) return EXL3_EINVAL;
    }
    Scratch& S = tls;
    if ((int64_t)S.count.size() < n) S.count.assign(n, 0);

    // 1-2
    for (int64_t i = 0; i < n; ++i)
        if (view[i] == 1 && res[i] == 0) {
            res[i] = 1;
            age[i] = tick;
        }
    for (int64_t i = 0; i < n_done; ++i) {
        res[done[i]] = 1;
        age[done[i]] = tick;
        inflight[done[i]] = 0;
    }
    // 3
    st->ring_overflow += overflow;
    S.touched.clear();
    S.want.clear();
    if (newm > 0) {
        for (int64_t i = 0; i < newm; ++i) {
            const int64_t key = ring[1 + pos_of(i)];
            if (S.count[key]++ == 0) S.touched.push_back(key);
        }
        for (int64_t key : S.touched)
            if (res[key] == 0 && !inflight[key]) S.want.push_back(key);
        const int32_t* c = S.count.data();
        std::sort(S.want.begin(), S.want.end(),
                  [c](int64_t a, int64_t b) { return c[a] != c[b] ? c[a] > c[b] : a < b; });
        for (int64_t t : S.touched) S.count[t] = 0;
        st->masked += newm;
    }
    st->ring_seen = (int64_t)cnt;                // in [0, 2^32)
    // 4
    int64_t n_res = 0, n_inf = 0;
    for (int64_t i = 0; i < n; ++i) {
        n_res += res[i] != 0;
        n_inf += inflight[i] != 0;
    }
    const int64_t nwant = (int64_t)S.want.size();
    int64_t over = n_res + n_inf + nwant - st->budget, ne = 0;
    if (over > 0) {
        S.cand.clear();
        for (int64_t i = 0; i < n; ++i)
            if (res[i] && slot_of[i] >= 0 && !pin[i]) S.cand.push_back(i);
        const int64_t t1 = smallest_by_age(S.cand, age, over, ev);
        for (int64_t i = 0; i < t1; ++i) res[ev[i]] = 0;
        ne = t1;
        over -= t1;
        if (over > 0) {
            S.cand.clear();
            for (int64_t i = 0; i < n; ++i)
                if (res[i] && !pin[i] && age[i] <= tick - st->admit_age) S.cand.push_back(i);
            const int64_t t2 = smallest_by_age(S.cand, age, over, ev + t1);
            for (int64_t i = t1; i < t1 + t2; ++i) res[ev[i]] = 0;
            ne += t2;
        }
        st->evicts += ne;
        n_res -= ne;
    }
    // 5
    const int64_t free_n = std::min(st->budget - n_res - n_inf, st->admit_qmax - n_inf);
    const int64_t na = std::max<int64_t>(0, std::min(free_n, nwant));
    for (int64_t i = 0; i < na; ++i) {
        adm[i] = S.want[i];
        inflight[adm[i]] = 1;
    }
    st->admit_dropped += nwant - na;
    // 6
    int64_t nd = 0;
    for (int64_t i = 0; i < n; ++i)
        if (res[i] != view[i]) {
            diff[nd] = i;
            vals[nd++] = res[i];
        }
    *n_adm = na;
    *n_ev = ne;
    *n_diff = nd;
    return EXL3_OK;
}
