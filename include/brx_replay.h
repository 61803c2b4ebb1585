/* libbrx_replay: eviction-policy replay over routing traces (host-only C++).
 *
 * Replaces the reference's Python trace tools for hit-rate studies:
 * simulate / belady / evaluate (bigrig_engine/pool.py:252-358) and the replay loop
 * select_policy runs per candidate (pool.py:219-249). Same contract as simulate(): a request
 * to a resident expert is a hit and touches it; a miss evicts victim() when the cache holds
 * `capacity` experts, then admits. No GPU involved. */
#ifndef BRX_REPLAY_H
#define BRX_REPLAY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BRX_REPLAY_OK      0
#define BRX_REPLAY_EINVAL  1

#define BRX_POLICY_LRU     0  /* least recently used (pool.py:53-72) */
#define BRX_POLICY_LFUDA   1  /* LFU with dynamic aging (policies/lfuda.py:67-161) */
#define BRX_POLICY_BELADY  2  /* optimal offline bound, furthest next use (pool.py:282-316) */
#define BRX_POLICY_WLFU    3  /* fewest uses in the last 128 requests (pool.py:75-118)       */
#define BRX_POLICY_S3FIFO  4  /* S3-FIFO, 10% probation, ghost ids (policies/s3fifo.py)      */
#define BRX_POLICY_ARC     5  /* adaptive replacement cache (policies/arc.py)                */
#define BRX_POLICY_LIRS    6  /* LIRS, 5% HIR, history 25% of capacity (policies/lirs.py)    */
#define BRX_POLICY_GATERANK 7 /* recency + 16 x linear top-8 rank bonus (policies/gaterank.py) */
#define BRX_POLICY_COACT   8  /* self-use + windowed co-activation (policies/coact.py)       */

/* LFUDA knobs (policies/lfuda.py:75-101): credit(rank) = 1 + rank_weight / (1 + rank)
 * (1 when rank_weight is 0); count saturates at fcap (no cap when fcap <= 0); an evicted
 * expert keeps count * ghost_decay when keep_ghost, else forgets it. */
typedef struct brx_lfuda_params {
    double rank_weight;
    double fcap;
    double ghost_decay;
    int32_t keep_ghost;
    int32_t reserved;
} brx_lfuda_params;

const char* brx_replay_last_error(void);
/* The shipped defaults: rank_weight 0, fcap 12, ghost_decay 0.5, keep_ghost 1. */
void brx_lfuda_defaults(brx_lfuda_params* p);

/* Misses of one request sequence (simulate(), pool.py:252-279; belady(), pool.py:282-316).
 * seq [n] expert ids in [0, n_experts); ranks [n] router ranks or NULL (all 0); lfuda NULL =
 * defaults (ignored by the other policies). */
int brx_replay(int policy, const int32_t* seq, const int32_t* ranks, int64_t n, int capacity,
               int n_experts, const brx_lfuda_params* lfuda, int64_t* out_misses);

/* Misses of every (capacity, layer) cell of a routing trace idx [n_layers, n_tokens, k] (int32,
 * a layer's requests in router-rank order within each token, rank = position in the token;
 * pool.py:337-358): out_misses [n_caps, n_layers]. The cells run on `threads` threads
 * (<= 0: one per hardware thread). evaluate()'s mean miss rate per capacity is
 * sum over layers of misses / (n_layers * n_tokens * k). */
int brx_replay_trace(int policy, const int32_t* idx, int n_layers, int n_tokens, int k,
                     const int32_t* capacities, int n_caps, int n_experts,
                     const brx_lfuda_params* lfuda, int threads, int64_t* out_misses);

#ifdef __cplusplus
}
#endif
#endif /* BRX_REPLAY_H */
