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
// furthest away; exact, from precomputed next-use positions and an ordered set. The rest of the
// reference's zoo (windowed LFU, S3-FIFO, ARC, LIRS, gaterank, coact; pool.py:75-118 and
// policies/*.py) runs under the same contract in its shipped configuration.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <deque>
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

// ---------------------------------------------------------------------------- the rest of the
// policy zoo, each in its shipped configuration. Ordered lists are a membership code per
// expert plus the clock value at which it entered the list's newest end: the oldest member of
// a list is the smallest such value (E <= a few hundred, so a scan is cheap).
struct Lists {
    std::vector<int8_t> where;
    std::vector<int64_t> since;
    std::vector<int> size;
    int64_t clock = 0;
    Lists(int E, int n) : where(E, 0), since(E, 0), size(n + 1, 0) {}
    void put(int e, int lst) {
        --size[where[e]];
        ++size[lst];
        where[e] = (int8_t)lst;
        since[e] = ++clock;
    }
    int oldest(int lst) const {
        if (!size[lst]) return -1;
        int best = -1;
        for (int e = 0; e < (int)where.size(); ++e)
            if (where[e] == lst && (best < 0 || since[e] < since[best])) best = e;
        return best;
    }
};

// Fewest uses among the last 128 requests, ties to the least recent (pool.py:75-118).
struct Wlfu {
    int window = 128;
    std::vector<int64_t> uses, last;
    std::vector<char> held;
    std::vector<int32_t> recent;      // ring of the window's requests
    size_t head = 0, count = 0;
    int64_t tick = 0;
    explicit Wlfu(int E) : uses(E, 0), last(E, 0), held(E, 0), recent(128, 0) {}
    void use(int e) {
        last[e] = ++tick;
        if (count == (size_t)window) {
            --uses[recent[head]];
            recent[head] = e;
            head = (head + 1) % window;
        } else {
            recent[(head + count++) % window] = e;
        }
        ++uses[e];
    }
    void admit(int e, int) { held[e] = 1; use(e); }
    void touch(int e, int) { use(e); }
    int victim() const {
        int best = -1;
        for (int e = 0; e < (int)held.size(); ++e)
            if (held[e] && (best < 0 || uses[e] < uses[best] || (uses[e] == uses[best] && last[e] < last[best])))
                best = e;
        return best;
    }
    void evicted(int e) { held[e] = 0; }
};

// S3-FIFO (policies/s3fifo.py): lists 1 probationary S, 2 main M, 3 ghost ids G; hit counter
// capped at 3; victim() takes its expert out of its queue itself.
struct S3fifo {
    enum { S = 1, M = 2, G = 3 };
    Lists q;
    std::vector<int> hits;
    int s_target, ghost_max;
    S3fifo(int C, int E) : q(E, 3), hits(E, 0) {
        s_target = std::max(1, (int)std::nearbyint(0.10 * C));   // round half to even
        ghost_max = std::max(1, (int)std::nearbyint(1.0 * C));
    }
    void admit(int e, int) {
        if (q.where[e] == S || q.where[e] == M) return;
        hits[e] = 0;
        q.put(e, q.where[e] == G ? M : S);
    }
    void touch(int e, int) {
        if (hits[e] < 3) ++hits[e];
    }
    int victim() {
        while (q.size[S] || q.size[M]) {
            if (q.size[S] >= s_target || !q.size[M]) {
                const int e = q.oldest(S);
                if (hits[e] > 1) {
                    hits[e] = 0;
                    q.put(e, M);
                    continue;
                }
                hits[e] = 0;
                q.put(e, G);
                if (q.size[G] > ghost_max) q.put(q.oldest(G), 0);
                return e;
            }
            const int e = q.oldest(M);
            if (hits[e] > 0) {
                --hits[e];
                q.put(e, M);
                continue;
            }
            hits[e] = 0;
            q.put(e, 0);
            return e;
        }
        return -1;
    }
    void evicted(int e) {
        hits[e] = 0;
        if (q.where[e] == S || q.where[e] == M) q.put(e, 0);
    }
};

// ARC (policies/arc.py): lists 1 T1, 2 T2, 3 B1, 4 B2; the target size of T1 moves on a ghost
// hit at admission.
struct Arc {
    enum { T1 = 1, T2 = 2, B1 = 3, B2 = 4 };
    Lists q;
    int c;
    double target = 0.0;
    Arc(int C, int E) : q(E, 4), c(C) {}
    void trim() {
        auto& n = q.size;
        while (n[T1] + n[B1] > c && n[B1]) q.put(q.oldest(B1), 0);
        while (n[T1] + n[T2] + n[B1] + n[B2] > 2 * c) {
            if (n[B2]) q.put(q.oldest(B2), 0);
            else if (n[B1]) q.put(q.oldest(B1), 0);
            else break;
        }
    }
    void admit(int e, int) {
        auto& n = q.size;
        const int w = q.where[e];
        if (w == B1) {
            target = std::min((double)c, target + std::max(1.0, (double)n[B2] / (double)std::max(1, n[B1])));
            q.put(e, T2);
        } else if (w == B2) {
            target = std::max(0.0, target - std::max(1.0, (double)n[B1] / (double)std::max(1, n[B2])));
            q.put(e, T2);
        } else {
            q.put(e, T1);
        }
        trim();
    }
    void touch(int e, int) { q.put(e, T2); }
    int victim() const {
        const auto& n = q.size;
        if (n[T1] && ((double)n[T1] > target || !n[T2])) return q.oldest(T1);
        if (n[T2]) return q.oldest(T2);
        return -1;
    }
    void evicted(int e) {
        if (q.where[e] == T1) q.put(e, B1);
        else if (q.where[e] == T2) q.put(e, B2);
        trim();
    }
};

// LIRS (policies/lirs.py): 5% of capacity (at least 1) for resident HIR experts, non-resident
// history in the stack bounded to 25% of capacity.
struct Lirs {
    enum { LIR = 1, HIR = 2 };
    int hir_slots, lir_slots, hist_slots;
    std::vector<int8_t> status;
    std::vector<char> held, in_s, in_q;
    std::vector<int64_t> s_at, q_at;
    int n_lir = 0, n_ghost = 0;
    int64_t clock = 0;
    Lirs(int C, int E)
        : status(E, 0), held(E, 0), in_s(E, 0), in_q(E, 0), s_at(E, 0), q_at(E, 0) {
        const int h = std::max(1, (int)std::nearbyint(0.05 * C));
        hir_slots = std::max(1, std::min(h, C - 1));
        lir_slots = C - hir_slots;
        hist_slots = std::max(1, (int)std::nearbyint(0.25 * C));
    }
    int E() const { return (int)status.size(); }
    void s_push(int e) { in_s[e] = 1; s_at[e] = ++clock; }
    void q_push(int e) { in_q[e] = 1; q_at[e] = ++clock; }
    int s_bottom(bool nonresident_only = false) const {
        int best = -1;
        for (int e = 0; e < E(); ++e)
            if (in_s[e] && (!nonresident_only || !held[e]) && (best < 0 || s_at[e] < s_at[best])) best = e;
        return best;
    }
    void prune() {
        for (;;) {
            const int b = s_bottom();
            if (b < 0 || status[b] == LIR) return;
            in_s[b] = 0;
            if (!held[b]) {
                status[b] = 0;
                --n_ghost;
            }
        }
    }
    void trim_history() {
        while (n_ghost > hist_slots) {
            const int b = s_bottom(true);
            if (b < 0) {
                n_ghost = 0;
                return;
            }
            in_s[b] = 0;
            status[b] = 0;
            --n_ghost;
        }
    }
    void make_lir(int e) {
        status[e] = LIR;
        ++n_lir;
        s_push(e);
        in_q[e] = 0;
        while (n_lir > lir_slots) {
            prune();
            const int b = s_bottom();
            if (b < 0) break;
            in_s[b] = 0;
            status[b] = HIR;
            --n_lir;
            if (held[b]) q_push(b);
            prune();
        }
        prune();
    }
    void admit(int e, int) {
        const bool found = in_s[e];
        if (found && !held[e]) --n_ghost;
        held[e] = 1;
        if (found) {
            make_lir(e);
        } else if (n_lir < lir_slots) {
            status[e] = LIR;
            ++n_lir;
            s_push(e);
        } else {
            status[e] = HIR;
            s_push(e);
            q_push(e);
        }
    }
    void touch(int e, int) {
        if (status[e] == LIR) {
            const bool was_bottom = s_bottom() == e;
            s_push(e);
            if (was_bottom) prune();
        } else if (in_s[e]) {
            make_lir(e);
        } else {
            s_push(e);
            q_push(e);
        }
    }
    int victim() {
        int best = -1;
        for (int e = 0; e < E(); ++e)
            if (in_q[e] && (best < 0 || q_at[e] < q_at[best])) best = e;
        if (best >= 0) return best;
        prune();
        for (int e = 0; e < E(); ++e)
            if (in_s[e] && held[e] && (best < 0 || s_at[e] < s_at[best])) best = e;
        if (best >= 0) return best;
        for (int e = 0; e < E(); ++e)
            if (held[e]) return e;
        return -1;
    }
    void evicted(int e) {
        held[e] = 0;
        in_q[e] = 0;
        if (status[e] == LIR) {
            --n_lir;
            in_s[e] = 0;
            status[e] = 0;
        } else if (in_s[e]) {
            ++n_ghost;
        }
        prune();
        trim_history();
    }
};

// gaterank (policies/gaterank.py): key = max(old key, tick + 16 w(rank)), w linear over top-8,
// victim = lowest (key, expert id).
struct GateRank {
    double boost = 16.0;
    int k = 8;
    std::vector<double> key;
    std::vector<char> has;
    int64_t ticks = 0;
    explicit GateRank(int E) : key(E, 0.0), has(E, 0) {}
    double w(int r) const { return k <= 1 ? 1.0 : std::max(0.0, (double)(k - 1 - r) / (double)(k - 1)); }
    void use(int e, int r) {
        ++ticks;
        double v = (double)ticks + boost * w(r);
        if (has[e] && key[e] > v) v = key[e];
        key[e] = v;
        has[e] = 1;
    }
    void admit(int e, int r) { use(e, r); }
    void touch(int e, int r) { use(e, r); }
    int victim() const {
        int best = -1;
        for (int e = 0; e < (int)key.size(); ++e)
            if (has[e] && (best < 0 || key[e] < key[best])) best = e;
        return best;
    }
    void evicted(int e) { has[e] = 0; }
};

// coact (policies/coact.py): score = decayed self-use + 0.8 x windowed co-activation affinity
// (half-life 128 requests, window 12, at most 64 partners kept per expert when more than 128
// are seen, support floor 4); victim = lowest (score, last use). Values are stored times a
// growth factor g instead of decaying every value per request. Tokens are recognised from the
// rank stream: a rank not above the previous one opens a new token.
struct CoAct {
    double decay, beta = 0.8;
    int window = 12, max_nb = 64, min_support = 4;
    int E;
    std::vector<char> held;
    std::vector<double> selfuse, affinity;
    std::vector<int64_t> last, tokens;
    std::vector<std::vector<std::pair<int, int64_t>>> partners;   // first-seen order
    std::vector<int32_t> slot_of;                                   // [E * E]: index in partners
    double g = 1.0;
    int64_t t = 0;
    std::vector<int> token;
    int prev_rank = 1 << 30;
    struct Entry {
        int e;
        double g;
        std::vector<std::pair<int, double>> given;   // first-granted order
    };
    std::deque<Entry> recent;
    explicit CoAct(int E_)
        : E(E_), held(E_, 0), selfuse(E_, 0.0), affinity(E_, 0.0), last(E_, 0), tokens(E_, 0),
          partners(E_), slot_of((size_t)E_ * E_, -1) {
        decay = std::pow(0.5, 1.0 / 128.0);
    }
    int64_t count(int y, int x) const {
        const int32_t i = slot_of[(size_t)y * E + x];
        return i < 0 ? 0 : partners[y][i].second;
    }
    void bump(int a, int b) {
        int32_t& i = slot_of[(size_t)a * E + b];
        if (i < 0) {
            i = (int32_t)partners[a].size();
            partners[a].push_back({b, 0});
        }
        ++partners[a][i].second;
    }
    int64_t support(int y) const { return tokens[y] > min_support ? tokens[y] : min_support; }
    void end_token() {
        const int n = (int)token.size();
        for (int i = 0; i < n; ++i) {
            const int a = token[i];
            ++tokens[a];
            for (int j = i + 1; j < n; ++j) {
                bump(a, token[j]);
                bump(token[j], a);
            }
            auto& pa = partners[a];
            if ((int)pa.size() > 2 * max_nb) {   // keep the most frequent, ties in first-seen order
                std::stable_sort(pa.begin(), pa.end(),
                                 [](const std::pair<int, int64_t>& u, const std::pair<int, int64_t>& v) {
                                     return u.second > v.second;
                                 });
                for (auto& pr : pa) slot_of[(size_t)a * E + pr.first] = -1;
                pa.resize(max_nb);
                for (int q = 0; q < max_nb; ++q) slot_of[(size_t)a * E + pa[q].first] = q;
            }
        }
        token.clear();
    }
    void clock(int e, int rank) {
        if (rank <= prev_rank) end_token();
        prev_rank = rank;
        token.push_back(e);
        ++t;
        g /= decay;
        if (g > 1e120) {
            const double sc = g;
            for (int x = 0; x < E; ++x) {
                selfuse[x] /= sc;
                affinity[x] /= sc;
            }
            for (auto& en : recent) {
                en.g /= sc;
                for (auto& gv : en.given) gv.second /= sc;
            }
            g = 1.0;
        }
    }
    void grant(int e) {
        Entry en{e, g, {}};
        const double scale = g / (double)support(e);
        for (const auto& pr : partners[e]) {
            const int x = pr.first;
            if (x != e && held[x]) {
                const double v = (double)pr.second * scale;
                affinity[x] += v;
                en.given.push_back({x, v});
            }
        }
        recent.push_back(std::move(en));
        while ((int)recent.size() > window) {
            for (const auto& gv : recent.front().given)
                if (held[gv.first]) affinity[gv.first] -= gv.second;
            recent.pop_front();
        }
    }
    double seed(int e) {
        double total = 0.0;
        for (auto& en : recent) {
            if (en.e == e) continue;
            double v = 0.0;
            bool have = false;
            for (const auto& gv : en.given)
                if (gv.first == e) { v = gv.second; have = true; break; }
            if (!have) {
                const int64_t c = count(en.e, e);
                if (!c) continue;
                v = ((double)c / (double)support(en.e)) * en.g;
                en.given.push_back({e, v});
            }
            total += v;
        }
        return total;
    }
    void admit(int e, int r) {
        clock(e, r);
        held[e] = 1;
        affinity[e] = seed(e);
        selfuse[e] += g * 1.0;
        last[e] = t;
        grant(e);
        (void)r;
    }
    void touch(int e, int r) {
        clock(e, r);
        selfuse[e] += g * 1.0;
        last[e] = t;
        grant(e);
    }
    int victim() const {
        int best = -1;
        double bs = 0.0;
        for (int x = 0; x < E; ++x) {
            if (!held[x]) continue;
            const double sx = selfuse[x] + beta * affinity[x];
            if (best < 0 || sx < bs || (sx == bs && last[x] < last[best])) {
                best = x;
                bs = sx;
            }
        }
        return best;
    }
    void evicted(int e) {
        held[e] = 0;
        affinity[e] = 0.0;
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
        case BRX_POLICY_WLFU: {
            Wlfu p(E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_S3FIFO: {
            S3fifo p(C, E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_ARC: {
            Arc p(C, E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_LIRS: {
            Lirs p(C, E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_GATERANK: {
            GateRank p(E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
        case BRX_POLICY_COACT: {
            CoAct p(E);
            *out = run_policy(p, seq, ranks, n, C, E, in);
            return BRX_REPLAY_OK;
        }
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
    if (policy < BRX_POLICY_LRU || policy > BRX_POLICY_COACT) return fail("unknown policy");
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
