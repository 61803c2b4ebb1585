"""Write tests/golden/policy_zoo_vectors.npz: miss counts and victim sequences of the
reference's eviction-policy zoo on fixed request streams.

Nothing else in the reference pins these policies' decisions (its tests check only the cache
contract), so this script imports the reference's pure-Python policy modules -- they need no
MLX -- and replays the streams through them with the reference's own `simulate` contract
(bigrig_engine/pool.py:252-279), each policy resolved by the reference's `_policy_factory` (its
shipped configuration). Run once, in a container that has the reference checked out:

    python tests/golden/make_policy_vectors.py /root/reference

The output holds only data: the request streams, their router ranks, and per (policy, stream,
capacity) the miss count and the first victims.
"""
from __future__ import annotations

import os
import sys

import numpy as np

POLICIES = ("wlfu", "s3fifo", "arc", "lirs", "gaterank", "coact", "lfuda", "lru")
CAPACITIES = (4, 8, 16, 32, 38)
N_VICTIMS = 256
HERE = os.path.dirname(os.path.abspath(__file__))


def streams() -> dict:
    """name -> (E, experts [n], ranks [n]): token streams of top-k picks in rank order."""
    out = {}
    rng = np.random.default_rng(20261202)
    for name, E, k, T, skew in (("uniform_e32_k4", 32, 4, 300, 0.0),
                                ("zipf_e64_k8", 64, 8, 300, 1.1),
                                ("zipf_e128_k8", 128, 8, 250, 0.8),
                                ("zipf_e256_k8", 256, 8, 250, 1.1)):
        if skew:
            w = 1.0 / np.arange(1, E + 1) ** skew
            p = w[rng.permutation(E)]
            p = p / p.sum()
        else:
            p = None
        toks = [rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]
        out[name] = (E, np.concatenate(toks).astype(np.int16),
                     np.tile(np.arange(k, dtype=np.int8), T))
    idx = np.load(os.path.join(HERE, "qwen3_full.npz"))["idx"]
    for layer in (0, 17):
        seq = np.asarray(idx[layer, :400], dtype=np.int16).reshape(-1)
        out[f"qwen3_layer{layer}_400tok"] = (128, seq, np.tile(np.arange(8, dtype=np.int8), 400))
    return out


def replay(factory, seq, ranks, C, E):
    """simulate()'s loop, also recording the victims."""
    pol = factory(C, E)
    resident, misses, victims = set(), 0, []
    for e, r in zip(seq.tolist(), ranks.tolist()):
        if e in resident:
            pol.touch(e, r)
            continue
        misses += 1
        if len(resident) >= C:
            v = pol.victim()
            if v >= 0:
                resident.discard(v)
                if hasattr(pol, "evicted"):
                    pol.evicted(v)
            victims.append(v)
        resident.add(e)
        pol.admit(e, r)
    return misses, victims


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from bigrig_engine import pool as RP   # noqa: E402  (the reference, pure Python)
    data = {}
    for sname, (E, seq, ranks) in streams().items():
        data[f"{sname}/seq"] = seq
        data[f"{sname}/ranks"] = ranks
        data[f"{sname}/n_experts"] = np.array(E, dtype=np.int32)
        for name in POLICIES:
            for C in CAPACITIES:
                if C >= E:
                    continue
                fac = RP._policy_factory(name, C, E)
                m, vic = replay(fac, seq, ranks, C, E)
                ref = RP.simulate(seq.tolist(), C, E, fac, ranks.tolist())["misses"]
                assert m == ref, (name, sname, C, m, ref)
                data[f"{sname}/{name}/C{C}/misses"] = np.array(m, dtype=np.int64)
                data[f"{sname}/{name}/C{C}/victims"] = np.array(vic[:N_VICTIMS], dtype=np.int16)
    path = os.path.join(HERE, "policy_zoo_vectors.npz")
    np.savez_compressed(path, **data)
    print(f"wrote {path}: {len(data)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
