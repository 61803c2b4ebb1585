// Trace replay for expert-pool eviction policies, host-only C++ (libbrx_replay.so).
//
// The reference measures policies by replaying routing traces through a cache in Python
// (bigrig_engine/pool.py:219-358: simulate, belady, evaluate, select_policy). The same replay
// here runs per (policy, capacity, layer) in native code, the cells of a sweep spread over
// threads. Semantics are those of the pool's simulate(): a request to a resident expert is a
// hit and touches it; a miss evicts victim() when the cache is full, then admits. Requests
// are a layer's routing flattened in router-rank order within each token (pool.py:337-358).
//
// LRU evicts the least recently admitted-or-touched expert (pool.py:53-72). LFUDA
// (policies/lfuda.py:67-161): count += credit(rank) saturating at fcap, key = L + count,
// victim = smallest (key, last-use tick), L rises to the evicted key, the evicted expert keeps
// count * ghost_decay. Belady (pool.py:282-316): evict the resident whose next request is
// furthest away; exact, from precomputed next-use positions and an ordered set.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <set>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "../../include/brx_replay.h"

namespace {

thread_local std::string t_err;

int fail(const char* msg) {
    t_err = msg;
    return BRX_REPLAY_EINVAL;
}

struct Lru {
    std::vector<int64_t> last;
    std::vector<int32_t> res;     // resident ids
    int64_t tick = 0;
    explicit Lru(int E) : last(E, 0) {}
    void use(int e) { last[e] = ++tick; }
    void admit(int e, int) { res.push_back(e); use(e); }
    void touch(int e, int) { use(e); }
    int victim() const {
        int best = -1;
        for (int e : res)
            if (best < 0 || last[e] < last[best]) best = e;
        return best;
    }
    void evicted(int e) { res.erase(std::find(res.begin(), res.end(), e)); }
};

struct Lfuda {
    brx_lfuda_params p;
    double L = 0.0;
    std::vector<double> cnt, key;
    std::vector<int64_t> last;
    std::vector<char> has_key;
    std::vector<int32_t> res;
    int64_t tick = 0;
    Lfuda(int E, const brx_lfuda_params& q) : p(q), cnt(E, 0.0), key(E, 0.0), last(E, 0), has_key(E, 0) {}
    double credit(int rank) const { return p.rank_weight == 0.0 ? 1.0 : 1.0 + p.rank_weight / (1.0 + rank); }
    void bump(int e, int rank) {
        last[e] = ++tick;
        double c = cnt[e] + credit(rank);
        if (p.fcap > 0.0 && c > p.fcap) c = p.fcap;
        cnt[e] = c;
        key[e] = L + c;
        has_key[e] = 1;
    }
    void admit(int e, int rank) {
        res.push_back(e);
        if (!p.keep_ghost) cnt[e] = 0.0;
        bump(e, rank);
    }
    void touch(int e, int rank) { bump(e, rank); }
    int victim() const {
        int best = -1;
        for (int e : res) {
            if (best < 0) { best = e; continue; }
            const double ka = has_key[e] ? key[e] : 0.0, kb = has_key[best] ? key[best] : 0.0;
            if (ka < kb || (ka == kb && last[e] < last[best])) best = e;
        }
        return best;
    }
    void evicted(int e) {
        const double k = has_key[e] ? key[e] : L;
        has_key[e] = 0;
        if (k > L) L = k;
        res.erase(std::find(res.begin(), res.end(), e));
        if (!p.keep_ghost) {
            cnt[e] = 0.0;
            last[e] = 0;
        } else if (p.ghost_decay != 1.0) {
            cnt[e] *= p.ghost_decay;
        }
    }
};

template <typename Pol>
int64_t run_policy(Pol& pol, const int32_t* seq, const int32_t* ranks, int64_t n, int C, int E,
                   std::vector<char>& in) {
    int64_t misses = 0, size = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int e = seq[i];
        const int r = ranks ? ranks[i] : 0;
        if (in[e]) {
            pol.touch(e, r);
            continue;
        }
        ++misses;
        if (size >= C) {
            const int v = pol.victim();
            if (v >= 0) {
                in[v] = 0;
                --size;
                pol.evicted(v);
            }
        }
        in[e] = 1;
        ++size;
        pol.admit(e, r);
    }
    (void)E;
    return misses;
}

int64_t run_belady(const int32_t* seq, int64_t n, int C, int E) {
    std::vector<int64_t> nxt(n), seen(E, n);
    for (int64_t i = n - 1; i >= 0; --i) {
        nxt[i] = seen[seq[i]];
        seen[seq[i]] = i;
    }
    std::vector<int64_t> due(E, -1);      // a resident's next request, or -1 when absent
    std::set<std::pair<int64_t, int>> order;
    int64_t misses = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int e = seq[i];
        if (due[e] >= 0) {
            order.erase({due[e], e});
            due[e] = nxt[i];
            order.insert({due[e], e});
            continue;
        }
        ++misses;
        if ((int64_t)order.size() >= C) {
            auto far = std::prev(order.end());
            due[far->second] = -1;
            order.erase(far);
        }
        due[e] = nxt[i];
        order.insert({due[e], e});
    }
    return misses;
}

int check_seq(const int32_t* seq, int64_t n, int E) {
    if (n < 0) return fail("n < 0");
    if (n > 0 && !seq) return fail("seq is NULL");
    if (E < 1) return fail("n_experts < 1");
    for (int64_t i = 0; i < n; ++i)
        if (seq[i] < 0 || seq[i] >= E) return fail("a request names an expert outside [0, n_experts)");
    return BRX_REPLAY_OK;
}

int replay_one(int policy, const int32_t* seq, const int32_t* ranks, int64_t n, int C, int E,
               const brx_lfuda_params& lp, int64_t* out) {
    std::vector<char> in(E, 0);
    switch (policy) {
        case BRX_POLICY_LRU: {
            Lru p(E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_LFUDA: {
            Lfuda p(E, lp);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_BELADY:
            *out = run_belady(seq, n, C, E);
            return BRX_REPLAY_OK;
        default:
            return fail("unknown policy");
    }
}

}  // namespace

extern "C" {

const char* brx_replay_last_error(void) { return t_err.c_str(); }

void brx_lfuda_defaults(brx_lfuda_params* p) {
    if (!p) return;
    p->rank_weight = 0.0;
    p->fcap = 12.0;
    p->ghost_decay = 0.5;
    p->keep_ghost = 1;
}

int brx_replay(int policy, const int32_t* seq, const int32_t* ranks, int64_t n, int capacity,
               int n_experts, const brx_lfuda_params* lfuda, int64_t* out_misses) {
    if (!out_misses) return fail("out_misses is NULL");
    if (capacity < 1) return fail("capacity < 1");
    int rc = check_seq(seq, n, n_experts);
    if (rc) return rc;
    brx_lfuda_params lp;
    brx_lfuda_defaults(&lp);
    if (lfuda) lp = *lfuda;
    return replay_one(policy, seq, ranks, n, capacity, n_experts, lp, out_misses);
}

int brx_replay_trace(int policy, const int32_t* idx, int n_layers, int n_tokens, int k,
                     const int32_t* capacities, int n_caps, int n_experts,
                     const brx_lfuda_params* lfuda, int threads, int64_t* out_misses) {
    if (!idx || !capacities || !out_misses) return fail("idx, capacities and out_misses are required");
    if (n_layers < 1 || n_tokens < 0 || k < 1 || n_caps < 1) return fail("empty trace shape");
    for (int c = 0; c < n_caps; ++c)
        if (capacities[c] < 1) return fail("capacity < 1");
    const int64_t per = (int64_t)n_tokens * k;
    int rc = check_seq(idx, per * n_layers, n_experts);
    if (rc) return rc;
    if (policy != BRX_POLICY_LRU && policy != BRX_POLICY_LFUDA && policy != BRX_POLICY_BELADY)
        return fail("unknown policy");
    brx_lfuda_params lp;
    brx_lfuda_defaults(&lp);
    if (lfuda) lp = *lfuda;
    // a layer's requests are already in router-rank order within each token: rank = i % k
    std::vector<int32_t> ranks(per);
    for (int64_t i = 0; i < per; ++i) ranks[i] = (int32_t)(i % k);
    const int cells = n_caps * n_layers;
    std::atomic<int> next(0);
    auto worker = [&]() {
        for (int c = next++; c < cells; c = next++) {
            const int ci = c / n_layers, l = c % n_layers;
            replay_one(policy, idx + per * l, ranks.data(), per, capacities[ci], n_experts, lp,
                       out_misses + c);
        }
    };
    int nt = threads > 0 ? threads : (int)std::thread::hardware_concurrency();
    nt = std::max(1, std::min(nt, cells));
    std::vector<std::thread> pool;
    for (int t = 1; t < nt; ++t) pool.emplace_back(worker);
    worker();
    for (auto& t : pool) t.join();
    return BRX_REPLAY_OK;
}

}  // extern "C"
