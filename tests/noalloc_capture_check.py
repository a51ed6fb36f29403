"""Fresh-process check of qk_matmul_noalloc's first call on a device coming under HIP graph capture.

Run by tests/test_zz_no_alloc.py as its own process, so that nothing in it has used the static
workspace before: weights are uploaded, then the very first qk_matmul_noalloc calls of the process
are captured into a graph (no qk_init_stream before).  The graph is replayed three times with eager
qk_matmul calls and synchronisations between the replays; every replay's outputs must equal
qk_matmul's on the same inputs bitwise (the same kernels and plans).  Cases: an int8-GEMV shape whose
plan combines K-slices through the combine slots, and a Q4_K shape the general GEMV serves (its
tile counters).  Prints one line per replay and exits 0 when all match.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from conftest import load_hiprt_module, load_qk_module  # noqa: E402
from oracle_lib import SEED_BASE, Oracle, T_Q6_K  # noqa: E402

# (type, k, n, m, fused): Q6_K K=17408 N=1024 splits K into slices (combine slots); the general
# kernel (fused = 0) at three tokens splits tiles between waves (tile counters)
CASES = [(T_Q6_K, 17408, 1024, 1, 1), (T_Q6_K, 17408, 5120, 3, 0)]


def main():
    hiprt, qkmod = load_hiprt_module(), load_qk_module()
    hip = hiprt.Hip()
    qk = qkmod.Lib()
    o = Oracle()
    o.init(4)
    stream = hip.stream_create()
    plans, items = [], []
    for i, (typ, k, n, m, fused) in enumerate(CASES):
        seed = SEED_BASE | (0xE0 + i)
        w = o.weights(typ, n, k, seed)
        x = o.normal(seed ^ 0x55, m * k).reshape(m, k)
        W = qk.upload(w, typ, k, n, 1, stream)
        qk.set_tuning("gemv_fused", fused)
        plans.append(qk.gemv_plan([W], False, m))
        qk.set_tuning("gemv_fused", 1)
        items.append((W, hiprt.Buf.of(hip, x), hiprt.Buf(hip, m * n * 4), hiprt.Buf(hip, m * n * 4), m, n, fused))
    kinds = sorted({p["kernel"] for p in plans})
    print(f"plans: {[(p['kernel'], p['slices']) for p in plans]}", flush=True)
    if kinds != [1, 2] or plans[0]["slices"] < 2:
        print("FAIL: the cases no longer cover a sliced int8 plan and the general kernel", flush=True)
        return 1
    hip.stream_sync(stream)
    hip.begin_capture(stream)
    for W, xd, yd, _, m, _, fused in items:
        qk.set_tuning("gemv_fused", fused)
        qk.matmul_noalloc(W, xd.ptr, m, yd.ptr, stream)
    qk.set_tuning("gemv_fused", 1)
    graph, gexec = hip.end_capture(stream)
    ok = True
    for rep in range(3):
        for item in items:
            item[2].fill_nan()
        hip.graph_launch(gexec, stream)
        hip.stream_sync(stream)
        for W, xd, yd, yr, m, n, fused in items:
            qk.set_tuning("gemv_fused", fused)
            qk.matmul(W, xd.ptr, m, yr.ptr, stream)  # eager work between the replays
            qk.set_tuning("gemv_fused", 1)
            hip.stream_sync(stream)
            a, b = yd.get(np.float32, (m, n)), yr.get(np.float32, (m, n))
            same = bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))
            ok &= same
            print(f"replay {rep} t{W.type} k{W.k} n{n} m{m}: {'equal' if same else 'DIFFERENT'}", flush=True)
    hip.graph_destroy(graph, gexec)
    for W, xd, yd, yr, _, _, _ in items:
        qk.free(W)
        xd.close()
        yd.close()
        yr.close()
    hip.stream_destroy(stream)
    print("OK" if ok else "FAIL", flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
