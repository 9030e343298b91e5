#!/usr/bin/env python3
"""Benchmark of the DeepSeek-V2 routed-expert MoE block on one MI355X.

Workload (the configuration the headline metric is quoted on): one int8 MoE
layer -- hidden 1280, 64 routed SwiGLU experts of width 896 (int8, fp32 scales
per 128-group along K), top-6 softmax gate, 2 shared bf16 experts (width 1792),
fp32 router -- at decode batch 1 and batch 8, on synthetic data: weights
N(0, 0.02) rounded to bf16 then quantised, hidden states RMSNorm(N(0, 1)).

Cold HBM: the timed steps rotate over 11 independently seeded layers (2.65 GB
of int8 stacks, the 11-layer decode stack) and over distinct token batches,
so the working set is far beyond the 256 MB Infinity Cache; a "warm" figure
repeats one layer and one batch.  A step is one MoE layer over one batch.  K
steps are captured in one HIP graph (launch-bound decode) and replayed once
between a synchronize and a synchronize; W warm-up steps run first.

Reported (one JSON line): the int8 B=1 layer's microseconds (``value``) with
B=1/B=8 HBM-roofline fractions, the 11-layer decode step at B=8, prefill T=512
(Zipf-skewed routing) and T=4096 (plus the adversarial all-on-experts-0..5
case) TFLOP/s against the bf16 MFMA peak, the bf16-weight decode, per-kernel
durations measured live with HIP events around each launch, and the CPU
oracle's restatement of the reference's CPU path timed on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from collections.abc import Callable
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "unlimited-ocr-max_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "int8 MoE layer µs & % HBM peak at decode B=1/8; prefill T=512 TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

E, H, F, N_SHARED, TOPK, GROUP = 64, 1280, 896, 2, 6, 128
FS = N_SHARED * F
LAYERS = 11
ZIPF_S = 1.1
ZIPF_SCALE = 0.75
PREFILL_4K_LAYERS = 4
XCDS, SIMDS = 8, 1024  # MI355X: 8 XCDs, 256 CUs x 4 SIMDs


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------- synthetic layers


def make_layer(seed: int, int8: bool, device: str):
    """One layer of seeded N(0, 0.02) weights (bf16), int8-quantised per 128-group when ``int8``."""
    import torch
    import uocr_moe

    g = torch.Generator(device=device).manual_seed(seed)

    def randn(shape):
        return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)

    w = {"gate.gate_score.weight": randn((E, H)).float()}
    for proj, shape in (("gate_proj", (E, F, H)), ("up_proj", (E, F, H)), ("down_proj", (E, H, F))):
        stack = randn(shape)
        if int8:
            q, s = uocr_moe.quantize_per_group(stack, GROUP)
            w[f"experts.{proj}"], w[f"experts.{proj}_scales"] = q, s
        else:
            w[f"experts.{proj}"] = stack
        del stack
    for proj, shape in (("gate_proj", (FS, H)), ("up_proj", (FS, H)), ("down_proj", (H, FS))):
        w[f"shared_experts.{proj}.weight"] = uocr_moe.kblocked(randn(shape))
    cfg = uocr_moe.MoeConfig(hidden_size=H, moe_intermediate_size=F, n_routed_experts=E, num_experts_per_tok=TOPK,
                             n_shared_experts=N_SHARED, int8_experts=int8, group_size=GROUP)
    return uocr_moe.MoE(cfg, w), w


def rmsnorm_rows(g, rows: int, device: str):
    import torch

    x = torch.randn((rows, H), generator=g, device=device, dtype=torch.float32)
    return (x / torch.sqrt(torch.mean(x.double() ** 2, dim=1, keepdim=True) + 1e-6).float()).contiguous()


# ---------------------------------------------------------------------------- algorithmic work


def expert_bytes(int8: bool) -> int:
    if int8:
        return 3 * F * H + 4 * (2 * F * (H // GROUP) + H * (F // GROUP))
    return 3 * F * H * 2


def decode_bytes(u: int, rows: int, int8: bool) -> int:
    """Weights of the u selected experts (each read once), the shared experts, the router, x in, out."""
    return u * expert_bytes(int8) + 3 * FS * H * 2 + E * H * 4 + 2 * rows * H * 4


def prefill_flops(T: int) -> float:
    return 2.0 * T * TOPK * 3 * F * H + 2.0 * T * 3 * FS * H + 2.0 * T * H * E


# ---------------------------------------------------------------------------- timing helpers


def graph_of(fn_steps):
    """A HIP graph of the given step callables, captured after one eager warm-up of each."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in fn_steps[: min(len(fn_steps), 3)]:
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fn_steps:
            fn()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, repeats: int = 5, warm_s: float = 0.0) -> float:
    """Median ms of one replay, each bracketed by synchronizes and timed with stream events; after
    untimed replays for warm_s seconds when asked (the prefill's MFMA load moves the shader clock:
    the first tenths of a second of it ran about 8 % slower than the steady state)."""
    import time

    import torch

    t_end = time.perf_counter() + warm_s
    while time.perf_counter() < t_end:
        graph.replay()
        torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        graph.replay()
        stop.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop))
    return statistics.median(times)


def kernel_times(fn_steps) -> dict[str, list[float]]:
    """Per-launch kernel durations (ms) of the steps run eagerly, by kernel name."""
    import torch
    from uocr_moe import _lib

    cap = 16 * len(fn_steps) + 16
    torch.cuda.synchronize()
    _lib.timing_begin(cap)
    for fn in fn_steps:
        fn()
    rows = _lib.timing_end(cap)
    out: dict[str, list[float]] = {}
    for name, ms in rows:
        out.setdefault(name, []).append(ms)
    return out


def fused_errors() -> int:
    """The persistent decode kernel's error word after everything queued so far (0: every bounded wait
    ended in time, so the timed launches computed real outputs)."""
    from uocr_moe import _lib

    return _lib.fused_errors()


# ---------------------------------------------------------------------------- benchmark parts


def bench_stack(layers, B: int, steps: int, device: str, seed: int) -> dict:
    """The MoE stack of one decode step: the 11 int8 layers chained through the residual stream,
    x_{l+1} = x_l + MoE_l(x_l) as the decoder's layers add it (so routing differs per layer and the batch's
    tokens stay distinct), ``steps // 11`` whole steps in one graph.  Two ways, the same bits: one
    persistent launch for the whole stack (``decode_stack``, the step's figures), and 11 ``decode_rows``
    launches with their residual adds (one small elementwise kernel each)."""
    import torch
    from uocr_moe import decode_stack

    g = torch.Generator(device=device).manual_seed(seed)
    x0 = rmsnorm_rows(g, B, device)
    ws = layers[0].workspace(B, prefill=False)
    u, x = [], x0
    for moe in layers:
        y, ids, _ = moe.decode_rows(x, workspace=ws, routing=True)
        x = x + y
        u.append(int(torch.unique(ids).numel()))
    same = bool(torch.equal(decode_stack(layers, x0), x))

    def chained():
        y = x0
        for moe in layers:
            y = y + moe.decode_rows(y, workspace=ws)

    def stacked():
        decode_stack(layers, x0)

    nsteps = max(1, steps // LAYERS)
    us_c = time_graph(graph_of([chained] * nsteps)) * 1e3 / nsteps
    us = time_graph(graph_of([stacked] * nsteps)) * 1e3 / nsteps
    errors = fused_errors()
    nbytes = sum(decode_bytes(ui, B, True) for ui in u)
    return {"rows": B, "layers": LAYERS, "us_per_step": round(us, 2), "tokens_per_s": round(B / (us * 1e-6), 1),
            "steps_in_graph": nsteps, "bytes_per_step": nbytes, "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "distinct_experts": u,
            "fused_errors": errors, "stack_bits_equal_chain": same,
            "chained_us_per_step": round(us_c, 2), "chained_tokens_per_s": round(B / (us_c * 1e-6), 1),
            "chain": "x_{l+1} = x_l + MoE_l(x_l) over the 11 layers, measured: one persistent launch "
                     "(uocr_moe_decode_stack); chained_* = 11 decode_rows launches + 11 residual adds"}


def bench_decode(layers, B: int, steps: int, warmup: int, int8: bool, device: str, seed: int) -> dict:
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    pool = [rmsnorm_rows(g, B, device) for _ in range(4 * LAYERS)]
    ws = layers[0].workspace(B, prefill=False)
    # the experts each (layer, batch) pair selects
    u_of = {}
    for i, x in enumerate(pool):
        _, ids, _ = layers[i % LAYERS].decode_rows(x, workspace=ws, routing=True)
        u_of[i] = int(torch.unique(ids).numel())
    plan = [(i % LAYERS, i % len(pool)) for i in range(steps)]
    fns = [lambda l=l, p=p: layers[l].decode_rows(pool[p], workspace=ws) for l, p in plan]
    wfns = [lambda l=l, p=p: layers[l].decode_rows(pool[p], workspace=ws) for l, p in plan[:warmup]]
    if wfns:
        graph_of(wfns).replay()
    graph = graph_of(fns)
    ms = time_graph(graph)
    errors = fused_errors()
    us = ms * 1e3 / steps
    total_bytes = sum(decode_bytes(u_of[p], B, int8) for _, p in plan)
    gbs = total_bytes / (ms * 1e-3) / 1e9
    # warm: one layer, one batch, repeated
    wgraph = graph_of([lambda: layers[0].decode_rows(pool[0], workspace=ws)] * min(steps, 4 * LAYERS))
    warm_us = time_graph(wgraph) * 1e3 / min(steps, 4 * LAYERS)
    errors += fused_errors()
    warm_gbs = decode_bytes(u_of[0], B, int8) / (warm_us * 1e-6) / 1e9
    # live per-kernel durations over one rotation (eager; events around each launch)
    kt = kernel_times([lambda l=l, p=p: layers[l].decode_rows(pool[p], workspace=ws) for l, p in plan[: 4 * LAYERS]])
    fused = kt.get("decode_fused", [])
    fused_bytes = [decode_bytes(u_of[p], B, int8) for _, p in plan[: len(fused)]]
    res = {
        "us_per_layer": round(us, 3),
        "tokens_per_s": round(B / (us * 1e-6), 1),
        "bytes_per_layer_avg": int(total_bytes / steps),
        "distinct_experts_avg": round(statistics.mean(u_of[p] for _, p in plan), 2),
        "hbm_gbs": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "warm_us_per_layer": round(warm_us, 3),
        "warm_gbs": round(warm_gbs, 1),
        "kernels_us_avg": {k: round(1e3 * statistics.mean(v), 3) for k, v in kt.items()},
        "kernel_sum_us_avg": round(1e3 * sum(sum(v) for v in kt.values()) / (4 * LAYERS), 3),
        "fused_errors": errors + fused_errors(),
    }
    if fused:
        res["fused_kernel"] = {
            "launches": len(fused),
            "avg_us": round(1e3 * statistics.mean(fused), 3),
            "avg_bytes": int(statistics.mean(fused_bytes)),
            "gbs": round(sum(fused_bytes) / (sum(fused) * 1e-3) / 1e9, 1),
        }
    return res


def bench_dense(N: int, K: int, device: str, rows=(1, 8), copies: int = 2, launches: int = 40) -> dict:
    """dense_bf16_qmv at one projection's shape (lm_head: 129280 x 1280): `copies` K-blocked bf16
    weights (2 x 331 MB > the 256 MB MALL, so each launch reads its weight cold), graph-timed."""
    import torch
    import uocr_moe

    g = torch.Generator(device=device).manual_seed(N + K)
    ws = [(torch.randn((K // 16, N, 16), generator=g, device=device) * 0.05).to(torch.bfloat16) for _ in range(copies)]
    out = {}
    for m in rows:
        xs = [torch.randn((m, K), generator=g, device=device) for _ in range(copies)]
        fns = [lambda i=i: uocr_moe.ops.dense_bf16_qmv(xs[i % copies], ws[i % copies]) for i in range(launches)]
        us = time_graph(graph_of(fns)) * 1e3 / launches
        nbytes = N * K * 2 + m * K * 4 + m * N * 4
        out[f"m{m}"] = {"us": round(us, 3), "bytes": nbytes, "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del ws
    torch.cuda.empty_cache()
    return out


def bench_ngram(device: str, rows: int = 8, vocab: int = 129280, window: int = 128, ngram: int = 35,
                copies: int = 64, launches: int = 64) -> dict:
    """ngram_block over `rows` x `vocab` logits (the decode step's guard, n = 35 over the 128-id window);
    `copies` logits buffers (265 MB, beyond the MALL) so each launch reads cold, graph-timed."""
    import torch
    import uocr_moe

    g = torch.Generator(device=device).manual_seed(35)
    logits = [torch.randn((rows, vocab), generator=g, device=device) for _ in range(copies)]
    outs = [torch.empty_like(x) for x in logits[:2]]
    motif = torch.randint(0, vocab, (rows, 40), generator=g, device=device, dtype=torch.int32)
    fill = torch.randint(0, vocab, (rows, window - 80), generator=g, device=device, dtype=torch.int32)
    history = torch.cat([motif, fill, motif], dim=1).contiguous()  # the last 34 ids recur: bans happen
    n = torch.tensor([ngram], dtype=torch.int32, device=device)
    fns = [lambda i=i: uocr_moe.ops.ngram_block(logits[i % copies], history, n, out=outs[i % 2])
           for i in range(launches)]
    us = time_graph(graph_of(fns)) * 1e3 / launches
    nbytes = 2 * rows * vocab * 4 + rows * window * 4
    del logits, outs
    torch.cuda.empty_cache()
    return {"rows": rows, "vocab": vocab, "window": window, "ngram": ngram, "us": round(us, 3), "bytes": nbytes,
            "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_attention(device: str, rows: int, attend: int = 640, layers: int = 12, heads: int = 10, head_dim: int = 128,
                    page_size: int = 128, sweeps: int = 4) -> dict:
    """paged_decode_attention at the served pool: 8 requests x 5 pages (512 prompt rows + the 128-row ring)
    plus the null page, 12 layers of 10 x 128 fp32 heads (645 MB, beyond the MALL).  `rows` requests attend
    `attend` rows each and append at row attend - 1; a graph walks the layers `sweeps` times, so every call
    reads its layer's rows cold."""
    import math

    import torch
    import uocr_moe

    per = math.ceil(attend / page_size)
    pages = 8 * per + 1
    g = torch.Generator(device=device).manual_seed(640)
    pool = torch.randn((pages, 2, layers, page_size, heads, head_dim), generator=g, device=device)
    order = torch.randperm(pages - 1, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    lut = torch.full((rows, per + 1), pages - 1, dtype=torch.int32)
    lut[:, :per] = order[: rows * per].reshape(rows, per)
    kv = uocr_moe.PagedKv(kv_blocks=pool, lookup_table=lut.to(device),
                          attend_lengths=torch.full((rows,), attend - 1, dtype=torch.int32, device=device),
                          attend_max=attend, write_index=torch.full((rows,), attend - 1, dtype=torch.int32,
                                                                    device=device))
    q, k_new, v_new = (torch.randn((rows, heads, head_dim), generator=g, device=device) for _ in range(3))
    out = torch.empty_like(q)
    from uocr_moe import _lib

    ws = torch.empty(_lib.load().uocr_paged_attention_workspace_bytes(rows, heads, attend) // 4 + 4,
                     device=device)
    scale = 1.0 / math.sqrt(head_dim)
    fns = [lambda l=l: uocr_moe.paged_decode_attention(q, k_new, v_new, kv=kv, layer_idx=l % layers, scale=scale,
                                                       out=out, workspace=ws)
           for l in range(layers * sweeps)]
    us = time_graph(graph_of(fns)) * 1e3 / len(fns)
    kt = kernel_times(fns[:layers])
    part_us = 1e3 * statistics.mean(kt["attn_partial"])
    nbytes = rows * heads * attend * head_dim * 4 * 2
    del pool, kv
    torch.cuda.empty_cache()
    return {"rows": rows, "attend": attend, "heads": heads, "head_dim": head_dim, "us_per_layer": round(us, 3),
            "partial_kernel_us": round(part_us, 3), "bytes": nbytes,
            "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "partial_hbm_frac": round(nbytes / (part_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_decoder_step(layers_w, B: int, device: str, steps: int = 20, attend: int = 640) -> dict:
    """The whole decode step (uocr_moe.Decoder.decode + lm_head) at the served shapes: 12 layers of 10 x 128
    attention over the paged pool (8 requests x 5 pages + the null page), layer 0's dense 6848 FFN, the 11
    int8 MoE layers built for the decode lines, lm_head 129 280.  B requests attend `attend` rows and append
    at row attend - 1.  `steps` decode steps in one graph, each from the same input hidden state."""
    import torch
    import uocr_moe

    hid, heads, hd, ffn, vocab, n_layers, page = H, 10, 128, 6848, 129280, LAYERS + 1, 128
    g = torch.Generator(device=device).manual_seed(777)

    def kb(n_out, k_in):
        w = (torch.randn((n_out, k_in), generator=g, device=device) * 0.02).to(torch.bfloat16)
        return uocr_moe.kblocked(w)

    w = {}
    for i in range(n_layers):
        p = f"layers.{i}."
        for c in "qkvo":
            w[f"{p}self_attn.{c}_proj.weight"] = kb(hid, hid)
        w[p + "input_layernorm.weight"] = 1 + 0.1 * torch.randn(hid, generator=g, device=device)
        w[p + "post_attention_layernorm.weight"] = 1 + 0.1 * torch.randn(hid, generator=g, device=device)
        if i == 0:
            w[p + "mlp.gate_proj.weight"], w[p + "mlp.up_proj.weight"] = kb(ffn, hid), kb(ffn, hid)
            w[p + "mlp.down_proj.weight"] = kb(hid, ffn)
        else:
            w.update({f"{p}mlp.{k}": v for k, v in layers_w[i - 1][1].items()})
    w["norm.weight"] = 1 + 0.1 * torch.randn(hid, generator=g, device=device)
    w["lm_head.weight"] = kb(vocab, hid)
    cfg = uocr_moe.DecoderConfig(hidden_size=hid, num_attention_heads=heads, num_hidden_layers=n_layers,
                                 intermediate_size=ffn, first_k_dense_replace=1, vocab_size=vocab,
                                 moe=layers_w[0][0].config)
    dec = uocr_moe.Decoder(cfg, w, max_seq_len=2048)
    per = (attend + page - 1) // page
    pages = 8 * per + 1
    pool = torch.randn((pages, 2, n_layers, page, heads, hd), generator=g, device=device)
    order = torch.randperm(pages - 1, generator=torch.Generator().manual_seed(2)).to(torch.int32)
    lut = torch.full((B, per + 1), pages - 1, dtype=torch.int32)
    lut[:, :per] = order[: B * per].reshape(B, per)
    kv = uocr_moe.PagedKv(kv_blocks=pool, lookup_table=lut.to(device),
                          attend_lengths=torch.full((B,), attend - 1, dtype=torch.int32, device=device),
                          attend_max=attend, write_index=torch.full((B,), attend - 1, dtype=torch.int32,
                                                                    device=device))
    positions = torch.full((B,), attend - 1, dtype=torch.int32, device=device)
    base = rmsnorm_rows(g, B, device)
    hidden = torch.empty_like(base)
    scratch = torch.empty_like(base)
    moe_ws = layers_w[0][0].workspace(B, prefill=False)
    from uocr_moe import _lib

    attn_ws = torch.empty(_lib.load().uocr_paged_attention_workspace_bytes(B, heads, attend) // 4, device=device)
    out = {}

    def step():
        hidden.copy_(base)
        out["logits"] = dec.logits_rows(dec.decode(hidden, positions=positions, kv=kv, moe_workspace=moe_ws,
                                                   attn_workspace=attn_ws, scratch=scratch))

    us = time_graph(graph_of([step] * steps)) * 1e3 / steps
    ok = bool(torch.isfinite(out["logits"]).all())
    del dec, w, pool, kv
    torch.cuda.empty_cache()
    return {"rows": B, "layers": n_layers, "attend": attend, "us_per_step": round(us, 2),
            "tokens_per_s": round(B / (us * 1e-6), 1), "steps_in_graph": steps, "finite": ok,
            "step": "12 x (norm, q/k/v, RoPE, paged attention, o_proj, norm, dense FFN or int8 MoE), norm, lm_head"}


def zipf_prefill_inputs(g, T: int, device: str, seed: int):
    """274 vision + 238 text rows of N(0,1) (per 512); a constant feature carries a Zipf(1.1) expert bias."""
    import torch

    x = torch.randn((T, H), generator=g, device=device, dtype=torch.float32)
    x[:, 0] = 1.0
    ranks = torch.randperm(E, generator=torch.Generator().manual_seed(seed)).double() + 1.0
    bias = (ZIPF_SCALE * -ZIPF_S * torch.log(ranks)).float().to(device)
    return x.contiguous(), bias


def prefill_setup(layers_w, T: int, device: str, seed: int, adversarial: bool = False):
    """``(moes, x, workspace)``: the layers with the Zipf bias (or the adversarial +10 on experts 0-5) in their
    router's column 0, and the T input rows whose constant feature carries it."""
    import torch
    import uocr_moe

    g = torch.Generator(device=device).manual_seed(seed)
    x, bias = zipf_prefill_inputs(g, T, device, seed)
    if adversarial:
        bias = torch.zeros(E, device=device)
        bias[:6] = 10.0
    moes = []
    for moe, w in layers_w:
        r = w["gate.gate_score.weight"].clone()
        r[:, 0] = bias
        moes.append(uocr_moe.MoE(moe.config, {**w, "gate.gate_score.weight": r}))
    return moes, x, moes[0].workspace(T, prefill=True)


def bench_prefill(layers_w, T: int, device: str, seed: int, adversarial: bool = False) -> dict:
    import torch

    moes, x, ws = prefill_setup(layers_w, T, device, seed, adversarial)
    hist = None
    touched = []
    for m in moes:
        _, ids, _ = m(x, workspace=ws, routing=True)
        counts = torch.bincount(ids.flatten().long(), minlength=E)
        touched.append(int((counts > 0).sum()))
        if hist is None:
            hist = counts.cpu().tolist()
    fns = [lambda m=m: m(x, workspace=ws) for m in moes]
    graph = graph_of(fns)
    ms = time_graph(graph, repeats=5, warm_s=0.3)
    us = ms * 1e3 / len(moes)
    flops = prefill_flops(T)
    tflops = flops / (us * 1e-6) / 1e12
    bytes_ = statistics.mean(t * expert_bytes(True) for t in touched) + 3 * FS * H * 2 + E * H * 4 + 2 * T * H * 4
    t_hbm = bytes_ / (HBM_PEAK_GBS * 1e9)
    t_mfma = flops / (BF16_PEAK_TFLOPS * 1e12)
    kt = kernel_times(fns)
    return {
        "tokens": T,
        "us_per_layer": round(us, 2),
        "tokens_per_s": round(T / (us * 1e-6), 1),
        "gflop": round(flops / 1e9, 3),
        "tflops": round(tflops, 2),
        "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
        "bytes_per_layer": int(bytes_),
        "hbm_gbs": round(bytes_ / (us * 1e-6) / 1e9, 1),
        "roofline_bound": "hbm" if t_hbm > t_mfma else "mfma",
        "roofline_frac": round(max(t_hbm, t_mfma) / (us * 1e-6), 4),
        "experts_touched_avg": round(statistics.mean(touched), 2),
        "expert_histogram_layer0": hist,
        "kernels_us_avg": {k: round(1e3 * statistics.mean(v), 2) for k, v in kt.items()},
    }


def cpu_model() -> str:
    """The host CPU's model name (lscpu), for the baseline record."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return "unknown"
    for line in out.splitlines():
        if line.startswith("Model name:"):
            return line.split(":", 1)[1].strip()
    return "unknown"


def bench_cpu_baseline(layer_int8, layer_bf16, budget_s: float, min_runs: int = 20) -> dict:
    """The reference's CPU decomposition (the oracle's restatement of the CPU path) on this host: the int8
    layer and its bf16 source layer, B=1 and B=8, on every host core and on one, medians of at least
    ``min_runs`` runs after a warm-up (about ``budget_s`` seconds in all)."""
    import numpy as np
    import torch

    from oracle import oracle as O

    def host(t):
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    def weights(w):
        w = {k: host(v) for k, v in w.items()}
        kw = dict(router=w["gate.gate_score.weight"], gate=w["experts.gate_proj"], up=w["experts.up_proj"],
                  down=w["experts.down_proj"], sh_gate=w["shared_experts.gate_proj.weight"],
                  sh_up=w["shared_experts.up_proj.weight"], sh_down=w["shared_experts.down_proj.weight"], topk=TOPK,
                  group=GROUP)
        if "experts.gate_proj_scales" in w:
            kw.update(gate_s=w["experts.gate_proj_scales"], up_s=w["experts.up_proj_scales"],
                      down_s=w["experts.down_proj_scales"])
        return O.MoeWeights(**kw)

    rng = np.random.default_rng(5)
    cores = O.threads(0)
    out = {"cores": cores, "model": cpu_model()}
    cases = [(kind, layer, B, t) for kind, layer in (("int8", weights(layer_int8)), ("bf16", weights(layer_bf16)))
             for B in (1, 8) for t in (cores, 1)]
    per_case = budget_s / len(cases)
    for kind, layer, B, threads in cases:
        x = O.rmsnorm_rows(rng, B, H)
        O.moe_decode_refdecomp(x, layer, threads=threads)  # warm-up
        times = []
        t_end = time.perf_counter() + per_case
        while time.perf_counter() < t_end or len(times) < min_runs:
            t0 = time.perf_counter()
            O.moe_decode_refdecomp(x, layer, threads=threads)
            times.append(time.perf_counter() - t0)
        key = f"{kind}_b{B}_{'all' if threads == cores else '1core'}"
        out[key] = {"us": round(1e6 * statistics.median(times), 1), "runs": len(times), "threads": threads}
    return out


# ---------------------------------------------------------------------------- HBM traffic (rocprofv3 --pmc)

COPY_ELEMS = 64 << 20  # the scale kernel: -x over 256 MiB of fp32 (reads 256 MiB, writes 256 MiB)


def traffic_probe() -> int:
    """Child mode run under ``rocprofv3 --pmc``: the int8 B=1 decode layer over the rotated layers (cold
    HBM, as in the timed region), then an elementwise kernel of known size that scales the counter."""
    import torch

    dev = "cuda:0"
    layers = [make_layer(1000 + l, True, dev)[0] for l in range(LAYERS)]
    g = torch.Generator(device=dev).manual_seed(1)
    xs = [rmsnorm_rows(g, 1, dev) for _ in range(LAYERS)]
    ws = layers[0].workspace(1, prefill=False)
    for i in range(2 * LAYERS):
        layers[i % LAYERS].decode_rows(xs[i % LAYERS], workspace=ws)
    src = torch.ones(COPY_ELEMS, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print("traffic probe done", flush=True)
    return 0


def run_counters(probe: str, counters: list[str], timeout_s: int = 150) -> list[tuple[int, str, dict]] | None:
    """One ``rocprofv3 --pmc`` pass over ``bench.py <probe>`` (a child process): per dispatch, in dispatch
    order, ``(dispatch id, kernel name, {counter: value summed over its instances})``."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        log("counters: rocprofv3 not found")
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = ["timeout", "-s", "KILL", str(timeout_s), prof, "--pmc", *counters, "--output-format", "csv", "-d", d,
               "-o", "pmc", "--", sys.executable, str(ROOT / "bench.py"), probe]
        log(f"counters: {' '.join(counters)} over {probe}")
        r = subprocess.run(cmd, capture_output=True, text=True, env={**os.environ, "TMPDIR": "/tmp"})
        path = Path(d) / "pmc_counter_collection.csv"
        if r.returncode != 0 and not path.exists():
            log(f"counters: pass failed ({r.returncode}): {r.stderr[-400:]}")
            return None
        per: dict[tuple[int, str], dict] = {}
        for row in csv.DictReader(open(path)):
            key = (int(row["Dispatch_Id"]), row["Kernel_Name"])
            c = per.setdefault(key, {})
            c[row["Counter_Name"]] = c.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    return [(k[0], k[1], v) for k, v in sorted(per.items())]


def measure_traffic(probe: str, kernels: dict[str, Callable[[list], list]]) -> dict | None:
    """HBM bytes per launch from two passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled so
    that the probe's closing elementwise kernel reads and writes its known 256 MiB.  ``kernels`` maps a
    label to a selector of that label's dispatches from the list of (id, name, counters)."""
    res: dict = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = run_counters(probe, [counter])
        if rows is None:
            return None
        scale = [c[counter] for _, n, c in rows if "neg" in n]
        if not scale:
            log(f"traffic: {counter}: no dispatches of the scale kernel")
            return None
        factor = COPY_ELEMS * 4 / 1024 / statistics.mean(scale)
        for label, pick in kernels.items():
            mine = [c[counter] for _, _, c in pick(rows)]
            if not mine:
                log(f"traffic: {counter}: no dispatches of {label}")
                return None
            r = res.setdefault(label, {})
            r[counter] = {"kib_per_launch": round(statistics.mean(mine), 1), "launches": len(mine),
                          "scale_kernel_kib": round(statistics.mean(scale), 1), "factor": round(factor, 4)}
    for label, r in res.items():
        fetch = r["FETCH_SIZE"]["kib_per_launch"] * r["FETCH_SIZE"]["factor"] * 1024
        write = r["WRITE_SIZE"]["kib_per_launch"] * r["WRITE_SIZE"]["factor"] * 1024
        r.update({"bytes": int(fetch + write), "fetch_bytes": int(fetch), "write_bytes": int(write)})
    return res


def _by_name(part: str) -> Callable[[list], list]:
    return lambda rows: [r for r in rows if part in r[1]]


def prefill_gemm_dispatches(rows: list) -> dict[str, list]:
    """The prefill probe's GEMM dispatches by workload, in its launch order: T=512 over the 11 layers, then
    T=4096 and the adversarial T=4096 over 4 layers each; gate/up and down alternate within a layer."""
    gemms = [r for r in rows if "k_moe_gemm" in r[1]]
    n512, n4k = 2 * LAYERS, 2 * PREFILL_4K_LAYERS
    groups = {"t512": gemms[:n512], "t4096": gemms[n512:n512 + n4k], "t4096_adversarial": gemms[n512 + n4k:]}
    out = {}
    for name, g in groups.items():
        out[f"{name}_gateup"] = g[0::2]
        out[f"{name}_down"] = g[1::2]
    return out


def prefill_probe() -> int:
    """Child mode run under ``rocprofv3 --pmc``: the bench's prefill workloads (T=512 with Zipf routing over
    the 11 layers, T=4096 and its adversarial case over 4), then the elementwise kernel that scales the
    traffic counters."""
    import torch

    dev = "cuda:0"
    layers_w = [make_layer(1000 + l, True, dev) for l in range(LAYERS)]
    for T, n, seed, adv in ((512, LAYERS, 512, False), (4096, PREFILL_4K_LAYERS, 4096, False),
                            (4096, PREFILL_4K_LAYERS, 4097, True)):
        moes, x, ws = prefill_setup(layers_w[:n], T, dev, seed, adv)
        for m in moes:
            m(x, workspace=ws)
        torch.cuda.synchronize()
        del moes, ws
    src = torch.ones(COPY_ELEMS, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print("prefill probe done", flush=True)
    return 0


def measure_prefill_counters(results: dict) -> dict | None:
    """MFMA utilisation and HBM traffic of the prefill GEMMs from rocprofv3 counters.

    * ``mfma_busy_frac`` = SQ_VALU_MFMA_BUSY_CYCLES (summed over every SIMD) / (GRBM_GUI_ACTIVE per XCC x
      1024 SIMDs): the fraction of the kernel's active cycles the matrix cores were busy.
    * ``mfma_flops`` = 512 x SQ_INSTS_VALU_MFMA_MOPS_BF16: the FLOPs the matrix cores executed, padded rows
      included (against the launch's algorithmic FLOPs).
    * ``bytes`` (FETCH_SIZE + WRITE_SIZE, scaled by the copy kernel).
    """
    rows = run_counters("--prefill-probe", ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                                            "GRBM_GUI_ACTIVE"])
    if rows is None:
        return None
    groups = prefill_gemm_dispatches(rows)
    out: dict = {}
    for label, disp in groups.items():
        if not disp:
            continue
        busy = [c["SQ_VALU_MFMA_BUSY_CYCLES"] / (c["GRBM_GUI_ACTIVE"] / XCDS * SIMDS) for _, _, c in disp]
        flops = [512.0 * c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] for _, _, c in disp]
        out[label] = {"launches": len(disp), "mfma_busy_frac": round(statistics.mean(busy), 4),
                      "mfma_flops_per_launch": round(statistics.mean(flops)),
                      "active_cycles_per_xcd": round(statistics.mean(c["GRBM_GUI_ACTIVE"] / XCDS for _, _, c in disp))}
    traffic = measure_traffic("--prefill-probe", {k: (lambda rows, k=k: prefill_gemm_dispatches(rows)[k])
                                                  for k in groups})
    if traffic is not None:
        for label, t in traffic.items():
            out.setdefault(label, {})["traffic_bytes"] = t["bytes"]
            out[label]["traffic"] = {k: t[k] for k in ("FETCH_SIZE", "WRITE_SIZE")}
    return out


# ---------------------------------------------------------------------------- main


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=440, help="timed decode layer-steps (one graph replay)")
    ap.add_argument("--warmup", type=int, default=44)
    ap.add_argument("--cpu-budget", type=float, default=16.0, help="seconds of CPU-baseline sampling")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="decode only (no prefill, no bf16)")
    ap.add_argument("--batches", default="1,8", help="int8 decode batches to time (1 is required)")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 --pmc traffic passes")
    ap.add_argument("--no-counters", action="store_true", help="skip the rocprofv3 --pmc passes over the prefill")
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--prefill-probe", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.traffic_probe:
        return traffic_probe()
    if args.prefill_probe:
        return prefill_probe()
    batches = sorted({int(b) for b in args.batches.split(",")})
    if 1 not in batches:
        print("--batches must include 1 (the headline workload)", file=sys.stderr)
        return 2
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the MoE block runs on a single MI355X here "
              "(run with --gpus 1; multi-GPU sharding is not part of this build)", file=sys.stderr)
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = "cuda:0"
    t_start = time.perf_counter()
    log(f"device {torch.cuda.get_device_name(0)}; building {LAYERS} int8 layers")
    layers_w = [make_layer(1000 + l, True, dev) for l in range(LAYERS)]
    layers = [m for m, _ in layers_w]
    torch.cuda.synchronize()
    results: dict = {}
    log("decode int8 B=1")
    results["decode_int8_b1"] = bench_decode(layers, 1, args.steps, args.warmup, True, dev, 1)
    log(f"  {results['decode_int8_b1']['us_per_layer']} us/layer")
    for B in batches:
        if B == 1:
            continue
        log(f"decode int8 B={B}")
        results[f"decode_int8_b{B}"] = bench_decode(layers, B, args.steps, args.warmup, True, dev, B)
        log(f"  {results[f'decode_int8_b{B}']['us_per_layer']} us/layer")
    for B in (1, 8):
        log(f"decode int8, the 11-layer MoE stack chained, B={B}")
        results[f"decode_int8_11layer_step_b{B}"] = bench_stack(layers, B, args.steps, dev, 11 + B)
        r = results[f"decode_int8_11layer_step_b{B}"]
        log(f"  {r['us_per_step']} us/step in one launch, {r['chained_us_per_step']} us/step as 11 launches")
    if not args.quick:
        for B in (1, 8):
            log(f"decode step, 12 layers + lm_head, B={B}")
            results[f"decoder_step_b{B}"] = bench_decoder_step(layers_w, B, dev)
            log(f"  {results[f'decoder_step_b{B}']}")
        log("prefill int8 T=512 (Zipf)")
        results["prefill_int8_t512"] = bench_prefill(layers_w, 512, dev, 512)
        log(f"  {results['prefill_int8_t512']['tflops']} TFLOP/s")
        log("prefill int8 T=4096")
        results["prefill_int8_t4096"] = bench_prefill(layers_w[:PREFILL_4K_LAYERS], 4096, dev, 4096)
        results["prefill_int8_t4096_adversarial"] = bench_prefill(layers_w[:PREFILL_4K_LAYERS], 4096, dev, 4097,
                                                                  adversarial=True)
        log(f"  {results['prefill_int8_t4096']['tflops']} / {results['prefill_int8_t4096_adversarial']['tflops']} TFLOP/s")
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        bf_src = make_layer(1000, False, dev)[1]  # the bf16 weights the first int8 layer was quantised from
        cpu = bench_cpu_baseline(layers_w[0][1], bf_src, args.cpu_budget)
        del bf_src
        log(f"  {cpu}")
    if not args.quick:
        del layers_w, layers
        torch.cuda.empty_cache()
        log("ngram_block, 8 x 129280 logits, n = 35 over 128 ids")
        results["ngram_block_b8"] = bench_ngram(dev)
        log(f"  {results['ngram_block_b8']}")
        log("paged_decode_attention, 640 rows attended, B=1/8")
        for B in (1, 8):
            results[f"paged_attention_b{B}"] = bench_attention(dev, B)
            log(f"  {results[f'paged_attention_b{B}']}")
        log("dense_bf16_qmv at lm_head's shape (129280 x 1280), M=1/8")
        results["dense_bf16_lm_head"] = bench_dense(129280, H, dev)
        log(f"  {results['dense_bf16_lm_head']}")
        log("decode bf16 B=1/8")
        bf = [make_layer(2000 + l, False, dev)[0] for l in range(LAYERS)]
        results["decode_bf16_b1"] = bench_decode(bf, 1, args.steps, args.warmup, False, dev, 101)
        results["decode_bf16_b8"] = bench_decode(bf, 8, args.steps, args.warmup, False, dev, 108)
        del bf

    b1 = results["decode_int8_b1"]
    fk = b1.get("fused_kernel", {})
    traffic = None
    if not args.no_traffic:
        t = measure_traffic("--traffic-probe", {"decode_fused": _by_name("k_decode_fused")})
        if t is not None:
            traffic = t["decode_fused"]
            results["traffic_decode_int8_b1"] = traffic
    if not args.quick and not args.no_counters:
        pc = measure_prefill_counters(results)
        if pc is not None:
            results["prefill_counters"] = pc
            for key, label in (("prefill_int8_t512", "t512"), ("prefill_int8_t4096", "t4096"),
                               ("prefill_int8_t4096_adversarial", "t4096_adversarial")):
                r = results.get(key)
                if r is None:
                    continue
                for kind, kname in (("gateup", "gemm_gateup"), ("down", "gemm_down")):
                    c = pc.get(f"{label}_{kind}")
                    us = r["kernels_us_avg"].get(kname)
                    if c is None or us is None:
                        continue
                    c["kernel_us"] = us
                    c["mfma_tflops_executed"] = round(c["mfma_flops_per_launch"] / (us * 1e-6) / 1e12, 1)
                    if "traffic_bytes" in c:
                        c["traffic_gbs"] = round(c["traffic_bytes"] / (us * 1e-6) / 1e9, 1)
                r["mfma_busy_frac"] = {k: pc[f"{label}_{k}"]["mfma_busy_frac"] for k in ("gateup", "down")
                                       if f"{label}_{k}" in pc}
    line = {
        "metric": METRIC,
        "value": b1["us_per_layer"],
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(b1["us_per_layer"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "int8 MoE decode layer, batch 1, 11 seeded layers rotated (cold HBM), HIP graph",
                   "hidden": H, "moe_ffn": F, "routed_experts": E, "top_k": TOPK, "shared_ffn": FS,
                   "group": GROUP, "batch": 1, "layers_rotated": LAYERS,
                   "operands": "int8 weights (fp32 per-128-group scales), fp32 activations and accumulation"},
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_fused (the whole int8 MoE layer in one persistent kernel), decode B=1",
            "achieved": fk.get("gbs"),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(fk["gbs"] / HBM_PEAK_GBS, 4) if fk else None,
            "traffic": None if traffic is None else traffic["bytes"],
            "algorithmic_bytes_per_launch": fk.get("avg_bytes"),
            "avg_launch_us": fk.get("avg_us"),
        },
        "cpu_baseline": None if cpu is None else {
            "value": cpu["int8_b1_all"]["us"], "unit": "us", "cores": cpu["cores"], "kind": "port",
            "sample": f"int8 decode layer B=1 on all {cpu['cores']} host threads ({cpu['model']}), median of "
                      f"{cpu['int8_b1_all']['runs']} runs; the reference's CPU decomposition restated in C. "
                      f"1 core: {cpu['int8_b1_1core']['us']} us; B=8: {cpu['int8_b8_all']['us']} us all cores, "
                      f"{cpu['int8_b8_1core']['us']} us 1 core; the bf16 layer (its unquantised source) B=1: "
                      f"{cpu['bf16_b1_all']['us']} / {cpu['bf16_b1_1core']['us']} us, B=8: "
                      f"{cpu['bf16_b8_all']['us']} / {cpu['bf16_b8_1core']['us']} us (all cores / 1 core)",
            "model": cpu["model"],
            "medians_us": {k: v for k, v in cpu.items() if k not in ("cores", "model")},
        },
        "results": results,
        "wall_s": round(time.perf_counter() - t_start, 1),
    }
    print(json.dumps(line), flush=True)
    failed = [k for k, r in results.items() if isinstance(r, dict) and r.get("fused_errors")]
    if failed:
        log(f"the persistent decode kernel reported failed waits in {failed}: those timings are not valid")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
