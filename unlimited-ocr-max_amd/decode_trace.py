"""Phase trace of one persistent decode launch (diagnostics, not part of the op).

    python unlimited-ocr-max_amd/decode_trace.py --build   # the traced library (UOCR_DECODE_TRACE=1)
    python unlimited-ocr-max_amd/decode_trace.py B          # one traced launch at batch B, on cuda:0

The traced build stamps each task's phases with the constant-rate wall clock
(100 MHz): start, weights landed (waited for only when tracing), inputs polled,
chains done, end, and when its wave learnt the routing; and each workgroup's
entry, epoch read and routing steps.  The launch traced is one of a stream of
back-to-back launches of one full-size int8 layer (the 64-expert, 1280/896
layer of bench.py), its weights warm in the MALL.  The stamps are global stores:
the traced launch runs about 3 µs longer than an untraced one.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
TRACE_LIB = HERE / "uocr_moe" / "trace" / "libuocr_moe.so"

KINDS = ["router", "sgu", "rgu", "sfold", "sdn", "rdn", "comb"]  # the kernel's task kinds, in order


def build() -> Path:
    sys.path.insert(0, str(HERE))
    import build as b

    TRACE_LIB.parent.mkdir(parents=True, exist_ok=True)
    return b.build(lib=TRACE_LIB, build_dir=HERE / "_build" / "trace", defines=("UOCR_DECODE_TRACE=1",))


def trace(B: int) -> None:
    os.environ["UOCR_MOE_LIB"] = str(TRACE_LIB)
    sys.path.insert(0, str(HERE.parent))
    sys.path.insert(0, str(HERE))
    import ctypes

    import numpy as np
    import torch

    import bench
    from uocr_moe import _lib

    dev = "cuda:0"
    moe = bench.make_layer(1, True, dev)[0]
    g = torch.Generator(device=dev).manual_seed(100 + B)
    xs = [bench.rmsnorm_rows(g, B, dev) for _ in range(4)]
    ws = moe.workspace(B, prefill=False)
    _, ids, _ = moe.decode_rows(xs[1], workspace=ws, routing=True)
    ng = int(torch.unique(ids).numel())
    nbuf = 1 << 17
    buf = torch.zeros(nbuf * 8, dtype=torch.int64, device=dev)
    gw = ctypes.c_int(0)
    for i in range(30):  # the traced launch follows a stream of launches (clocks up, caches steady)
        moe.decode_rows(xs[i % 4], workspace=ws)
    _lib.call("uocr_moe_fused_trace", buf.data_ptr(), buf.numel(), ctypes.byref(gw))
    moe.decode_rows(xs[1], workspace=ws)
    torch.cuda.synchronize()
    _lib.call("uocr_moe_fused_trace", buf.data_ptr(), buf.numel(), ctypes.byref(gw))  # reads the grid size back
    assert _lib.fused_errors() == 0
    tr = buf.cpu().numpy()
    wgs = gw.value // 12
    # the per-workgroup records follow the layout's task capacity (fused_layout's max_tasks)
    E, H, F, FS, K = bench.E, bench.H, bench.F, bench.FS, bench.TOPK
    gh, gf, gfs = H // 128, F // 128, FS // 128
    sub = 2 if B >= 4 else 1  # column blocks per routed int8 gate/up task (fused_sub)
    c_gu, c_dn = 64 // (2 * gh), 64 // gf
    per_gu, per_dn = -(-F // (c_gu * sub)), -(-H // c_dn)
    max_tasks = E + (FS // 64) * 2 * gh + (FS // 64) * B + (H // 64) * gfs + min(E, B * K) * (per_gu + per_dn) \
        + (H // 64) * B
    rec = tr.reshape(-1, 8)
    tasks, wg = rec[:max_tasks], rec[max_tasks:max_tasks + wgs]
    valid = tasks[:, 0] > 0
    t0 = min(tasks[valid, 0].min(), wg[wg[:, 6] > 0, 6].min())
    us = lambda v: (np.asarray(v, np.float64) - t0) / 100.0  # noqa: E731

    def q(v):
        v = np.asarray(v)
        return " - " if not len(v) else f"{np.percentile(v, 10):6.2f} {np.median(v):6.2f} {np.percentile(v, 90):6.2f}"

    print(f"B={B}, {ng} experts selected, {wgs} workgroups; microseconds from the first wave's start, "
          f"10th percentile / median / 90th over tasks")
    print(f"| task kind | tasks | start | weights landed | inputs polled | chains done | end |")
    print(f"|---|---:|---|---|---|---|---|")
    for k, name in enumerate(KINDS):
        blk = tasks[valid & (tasks[:, 6] == k)] if k else tasks[valid][: 64]
        if not len(blk):
            continue
        col = lambda i: us(blk[blk[:, i] > 0, i])  # noqa: E731
        print(f"| {name} | {len(blk)} | {q(us(blk[:, 0]))} | {q(col(1))} | {q(col(3))} | {q(col(4))} | {q(us(blk[:, 2]))} |")
    w = wg[wg[:, 0] > 0]
    print(f"| workgroup steps | {len(w)} | entry {q(us(w[:, 6]))} | epoch read {q(us(w[:, 7]))} | "
          f"logits seen {q(us(w[:, 1]))} | top-k {q(us(w[:, 5]))} | routing published {q(us(w[:, 2]))} |")
    print(f"| routing steps (token 0) | {len(w)} | logits seen {q(us(w[:, 1]))} | max {q(us(w[:, 3]))} | "
          f"exp sum {q(us(w[:, 4]))} | ranks {q(us(w[:, 5]))} | published {q(us(w[:, 2]))} |")


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--build":
        print(build())
    else:
        trace(int(sys.argv[1]) if len(sys.argv) > 1 else 1)
