#!/usr/bin/env python3
"""Benchmark of the 4-bit quantized matmul path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-cpu] [--profile [gemv|moe|gemm]]

Headline (BASELINE metric "4-bit GEMV achieved HBM GB/s at M=1"): one step is the
9B-class decode layer's six projections (q, k, v, o, gate_up, down)
at M=1 as the reference's engine runs them: q, k and v stacked into one matrix (its
attn.qkv tensor, one linear: src/engine.mm:1163-1167), so four launches of the decode
kernel (qkv, o, gate_up, down), 4-bit affine g64 with fp16 scales, weights
N(0, 0.02) quantized on the device and activations fp16 N(0, 1). Every step uses the next
of >= 1 GiB of distinct weight copies so that the 256 MB Infinity Cache cannot serve
re-reads. The steps are replayed from one HIP graph so that host launch cost does not pace
the GPU. value = algorithmic bytes of the step / measured time per step.

Also reported under "detail": the M=5 layer, the 27B layer at M=1 and M=8 (config 3), the
27B prefill layer at M=2048 (config 4, TFLOP/s against the dense fp16 MFMA peak), the MoE
layer at T=1 and T=512 (config 5), each projection's kernel time, the six-launch layer (q,
k, v as separate matrices), the native int15 MoE and linear, the 9B layer and the 27B
prefill with bf16 scales (the .rlm files' scale type), the output head at a vocabulary of
248,320, the engine's rl_mlp over .rlm files (dense 9B-shaped and the MoE layer) beside the
sum of its parts, a streaming probe of what this box's HBM delivers to plain read and copy
kernels (context for the roofline fractions, which stay against 8 TB/s), and the CPU
baseline: the reference's numpy dequant + fp32 matmul (oracle.linear_affine_cpu_f32) on a
bounded sample, timed on this host.

Timing: each entry captures one HIP graph of exactly --steps consecutive steps over its
rotating weight copies, replays it untimed (at least --warmup steps, and its first replay),
then times one replay with HIP events on the stream it runs on, queued directly behind one
more untimed replay so that the GPU does not idle before it.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, 2.5 PFLOP/s
CACHE_DEFEAT_BYTES = 1 << 30   # rotate >= 1 GiB of distinct weights


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def build_layer_copies(shapes, copies, seed, device, scale_dtype):
    from raceline_amd import synth

    layers = []
    for c in range(copies):
        layers.append([synth.random_affine(N, K, seed + 1000 * c + i, device, scale_dtype=scale_dtype)
                       for i, (_, K, N) in enumerate(shapes)])
    return layers


def layer_bytes(shapes, M):
    from raceline_amd.configs import linear_bytes

    return sum(linear_bytes(M, K, N) for _, K, N in shapes)


def copies_for(shapes):
    per = layer_bytes(shapes, 1)
    return max(2, -(-CACHE_DEFEAT_BYTES // per))


class StepGraphs:
    """Timing of an arbitrary step over rotating weight copies: step c runs steps_per_copy[c %
    n]. Every step runs once eagerly on a side stream (each call is valid before it is
    captured); time_steps then captures one HIP graph of exactly the timed number of
    consecutive steps and replays it on that stream, which the timing events bracket."""

    def __init__(self, steps_per_copy):
        import torch

        self.torch = torch
        self.fns = list(steps_per_copy)
        # The step's buffers come from the default stream's allocator pool, whose blocks may
        # still be written by kernels queued there (weight generation, freed temporaries).
        # The MoE step computes addresses from the routing tables it writes into such a
        # block: without this wait a queued kernel can overwrite them under the side stream.
        torch.cuda.synchronize()
        self.stream = torch.cuda.Stream()
        with torch.cuda.stream(self.stream):
            for fn in self.fns:
                fn()
        torch.cuda.synchronize()

    def graph_of(self, count):
        """One graph of `count` consecutive steps, starting at copy 0."""
        g = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(g, stream=self.stream):
            for i in range(count):
                self.fns[i % len(self.fns)]()
        return g


class LayerRunner(StepGraphs):
    """The layer's projections as one step: step c runs every projection on weight copy c."""

    def __init__(self, layers, shapes, M, device, kernel=0, outliers=0.0):
        import torch

        from raceline_amd import ops, synth

        self.layers, self.shapes, self.M = layers, shapes, M
        self.xs = {K: synth.random_activations(M, K, 7 + K, device, outliers) for _, K, _ in shapes}
        self.ys = [torch.empty((M, N), dtype=torch.float32, device=device) for _, _, N in shapes]
        self.kernel = kernel
        # grow the workspace to its largest size before capture (no allocation inside a graph)
        for (_, K, N) in shapes:
            ops._WS.get(device, ops.workspace_bytes(M, K, N))
        super().__init__([(lambda c=c: self.run_eager(c)) for c in range(len(layers))])

    def run_eager(self, c, only=None):
        from raceline_amd import ops

        for i, ((_, K, N), wt) in enumerate(zip(self.shapes, self.layers[c])):
            if only is not None and i != only:
                continue
            ops.linear(self.xs[K], wt, out=self.ys[i], kernel=self.kernel)


def timed_replay(g, stream, warm=1):
    """Seconds for one replay of the captured graph g on `stream`: `warm` untimed replays and
    a host synchronization, then one more untimed replay and, right behind it on the stream,
    the timed replay between two events, so that the GPU runs the timed replay with no idle
    gap before it (a short graph timed right after the host's synchronization ran at lower
    clocks: the 2 us norm of the engine entries read 4.9 us in graphs of 20 steps)."""
    import torch

    with torch.cuda.stream(stream):
        for _ in range(warm):
            g.replay()
        torch.cuda.synchronize()
        g.replay()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def time_steps(runner, steps, warmup):
    """Seconds per step: one captured graph of exactly `steps` consecutive steps, replayed
    max(1, ceil(warmup / steps)) times untimed (at least `warmup` steps, and the graph's first
    replay, which costs more than later ones), then timed (timed_replay)."""
    g = runner.graph_of(steps)
    t = timed_replay(g, runner.stream, max(1, -(-warmup // steps)))
    del g
    return t / steps      # seconds per step


MOE_EXPERT_BYTES = 1769472   # codes + fp16 s/b of one expert's gate_up [1024][2048] and down [2048][512]
MOE_T1_STEPS = 64            # distinct routings of the one-token MoE step


def moe_step_logits(T, E, copies, device):
    """Router logits for the MoE steps: one [T][E+1] matrix per step. A one-token step
    reads only its 9 experts (16 MB), so the same routing on every step of a copy would
    find them in the 256 MB Infinity Cache; at T = 1 each of MOE_T1_STEPS steps draws its
    own logits, so a round of steps touches several hundred MB per copy. At T = 512 a step
    reads every expert (more than the cache holds) and one routing serves every copy."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(601 + T)
    n = max(MOE_T1_STEPS, copies) if T == 1 else copies
    one = T > 1
    mats = [torch.randn((T, E + 1), generator=g, device=device, dtype=torch.float32) for _ in range(1 if one else n)]
    return [mats[0]] * n if one else mats


def moe_distinct_experts(logits, E, topk):
    """Distinct experts a step reads (its routed ones and the shared one), averaged over the
    steps' routings."""
    import torch

    from raceline_amd import ops

    seen = {}
    for lg in logits:
        key = id(lg)
        if key not in seen:
            seen[key] = int(torch.unique(ops.moe_route(lg, E, topk).sel).numel())
    vals = [seen[id(lg)] for lg in logits]
    return round(sum(vals) / len(vals), 2)


def bench_moe(device, steps, warmup):
    """the MoE layer (H=2048, E=256 + shared, I=512, top-8, norm_topk) at
    T=1 and T=512, all experts resident, >= 1 GiB of rotating weight copies. One step =
    route + gate/up (gather, SwiGLU fused) + down + combine into h. Bytes follow the
    algorithmic count distinct_experts * 1,769,472 + A*(2H*2 + 2I*4 + I*2 + H*4)."""
    import torch

    from raceline_amd import ops, synth
    from raceline_amd.configs import MOE

    E, H, I, topk = MOE["E"], MOE["H"], MOE["I"], MOE["topk"]
    per_copy = ops.packed_bytes(H, (E + 1) * 2 * I) + ops.packed_bytes(I, (E + 1) * H)
    copies = max(2, -(-CACHE_DEFEAT_BYTES // per_copy))
    log(f"[bench] building {copies} copies of the MoE experts ({per_copy / 1e6:.1f} MB each)")
    mws = []
    for c in range(copies):
        gu = synth.random_affine((E + 1) * 2 * I, H, 500 + 2 * c, device, packed=False)
        dn = synth.random_affine((E + 1) * H, I, 501 + 2 * c, device, packed=False)
        mws.append(ops.pack_moe(gu, dn, E, H, I))
        del gu, dn
    out = {}
    for T in MOE["tokens"]:
        x = synth.random_activations(T, H, 600 + T, device)
        logits = moe_step_logits(T, E, copies, device)
        h = torch.zeros((T, H), dtype=torch.float32, device=device)
        ws = torch.empty(ops.moe_workspace_bytes(T, E, topk, H, I), dtype=torch.uint8, device=device)
        fns = [(lambda mw=mws[j % copies], lg=lg: ops.moe(x, lg, mw, topk, h, workspace=ws))
               for j, lg in enumerate(logits)]
        sg = StepGraphs(fns)
        t = time_steps(sg, steps, warmup)
        distinct = moe_distinct_experts(logits, E, topk)
        A = T * (topk + 1)
        nbytes = int(round(distinct * MOE_EXPERT_BYTES)) + A * (2 * H * 2 + 2 * I * 4 + I * 2 + H * 4)
        flops = 2 * A * 3 * H * I
        out[f"moe_t{T}"] = {"us_per_step": round(t * 1e6, 2), "GB/s": round(nbytes / t / 1e9, 1),
                            "TFLOP/s": round(flops / t / 1e12, 2), "distinct_experts": distinct,
                            "algorithmic_bytes": nbytes}
        log(f"[bench] MoE T={T}: {t * 1e6:.1f} us/step, {nbytes / t / 1e9:.0f} GB/s ({distinct} experts)")
        del sg
    del mws
    torch.cuda.empty_cache()
    out.update(bench_moe_native(device, steps, warmup))
    return out


NATIVE_EXPERT_BYTES = 1585152   # int15 codes + fp32 row scales of one expert's gate_up [1024][2048] and down [2048][512]


def bench_moe_native(device, steps, warmup):
    """The same MoE layer in the reference's own expert format (kernels/linear.metal:254-308):
    native int15 codes with an fp32 scale per row, slot = expert, the down matrix's column
    scale applied in the SwiGLU. One step = route, gate_up product with the gather and the
    SwiGLU fused, down product, combine. Bytes: distinct_experts * 1,585,152 +
    A*(2H + 2*I*2 + 2*H*4) (x rows read; act and y each written and read once)."""
    import torch

    from raceline_amd import ops, synth
    from raceline_amd.configs import MOE

    E, H, I, topk = MOE["E"], MOE["H"], MOE["I"], MOE["topk"]
    per_copy = (E + 1) * NATIVE_EXPERT_BYTES
    copies = max(2, -(-CACHE_DEFEAT_BYTES // per_copy))
    log(f"[bench] building {copies} copies of the native MoE experts ({per_copy / 1e6:.1f} MB each)")
    stacks = []
    for c in range(copies):
        g = torch.Generator(device=device)
        g.manual_seed(700 + c)
        lo, hi = -(1 << 31), (1 << 31) - 1
        gw = torch.randint(lo, hi, ((E + 1) * 2 * I, H // 8), generator=g, device=device, dtype=torch.int32)
        dw = torch.randint(lo, hi, ((E + 1) * H, I // 8), generator=g, device=device, dtype=torch.int32)
        gs = torch.rand((E + 1) * 2 * I, generator=g, device=device) * 0.004 + 0.001
        ds = torch.rand((E + 1) * H, generator=g, device=device) * 0.004 + 0.001
        stacks.append((ops.pack_moe_native(gw, gs, 2 * I, "int15"), ops.pack_moe_native(dw, ds, H, "int15")))
        del gw, dw
    slots = torch.arange(E + 1, dtype=torch.int32, device=device)
    g = torch.Generator(device=device)
    g.manual_seed(800)
    cs = torch.rand(I, generator=g, device=device) + 0.5
    out = {}
    for T in MOE["tokens"]:
        x = synth.random_activations(T, H, 600 + T, device)
        logits = moe_step_logits(T, E, copies, device)
        h = torch.zeros((T, H), dtype=torch.float32, device=device)
        ws = torch.empty(ops.moe_workspace_bytes(T, E, topk, H, I), dtype=torch.uint8, device=device)
        fns = [(lambda st=stacks[j % copies], lg=lg: ops.moe_native(x, lg, st[0], st[1], slots, topk, h, cs=cs,
                                                                     workspace=ws))
               for j, lg in enumerate(logits)]
        sg = StepGraphs(fns)
        t = time_steps(sg, steps, warmup)
        distinct = moe_distinct_experts(logits, E, topk)
        A = T * (topk + 1)
        nbytes = int(round(distinct * NATIVE_EXPERT_BYTES)) + A * (2 * H + 2 * I * 2 + 2 * H * 4)
        out[f"moe_native_t{T}"] = {"us_per_step": round(t * 1e6, 2), "GB/s": round(nbytes / t / 1e9, 1),
                                   "distinct_experts": distinct, "algorithmic_bytes": nbytes, "book": "int15"}
        log(f"[bench] native MoE T={T}: {t * 1e6:.1f} us/step, {nbytes / t / 1e9:.0f} GB/s ({distinct} experts)")
        del sg
    del stacks
    torch.cuda.empty_cache()
    return out


def bench_native_epilogue(device, steps, warmup):
    """What the native linear's epilogue (the row scale) costs: linear_q4n against
    linear_q4n_raw (kernels/linear.metal:226-252), native int15 codes, on the 9B gate_up
    shape at M = 1 (over >= 1 GiB of copies) and the 27B gate_up at M = 2048."""
    import torch

    from raceline_amd import ops, synth

    out = {}
    for M, K, N in ((1, 4096, 24576), (2048, 5120, 34816)):
        per = K * N // 2 + 4 * N
        copies = max(2, -(-CACHE_DEFEAT_BYTES // per)) if M == 1 else 2
        g = torch.Generator(device=device)
        nws = []
        for c in range(copies):
            g.manual_seed(900 + c)
            w = torch.randint(-(1 << 31), (1 << 31) - 1, (N, K // 8), generator=g, device=device, dtype=torch.int32)
            nws.append(ops.pack_native(w, torch.rand(N, generator=g, device=device) * 0.01 + 0.001, "int15"))
            del w
        x = synth.random_activations(M, K, 901, device)
        y = torch.empty((M, N), dtype=torch.float32, device=device)
        ops._WS.get(device, ops.workspace_bytes(M, K, N))
        res = {}
        for name, fn in (("scaled", ops.linear_native), ("raw", ops.linear_native_raw)):
            sg = StepGraphs([(lambda nw=nw, fn=fn: fn(x, nw, out=y)) for nw in nws])
            t = time_steps(sg, steps if M == 1 else max(4, steps // 5), warmup if M == 1 else 2)
            res[name] = t
            del sg
        key = f"native_int15_k{K}_n{N}_m{M}"
        out[key] = {"scaled_us": round(res["scaled"] * 1e6, 2), "raw_us": round(res["raw"] * 1e6, 2),
                    "epilogue_share": round(1 - res["raw"] / res["scaled"], 4)}
        log(f"[bench] native linear {key}: {res['scaled'] * 1e6:.1f} us, raw {res['raw'] * 1e6:.1f} us")
        del nws
        torch.cuda.empty_cache()
    return {"native_epilogue": out}


HEAD_VOCAB = 248320           # the reference's Qwen3.5 vocabulary (tests/tiny_moe.py:121)


def bench_bf16(device, steps, warmup):
    """What real files run: tools/convert.py stores the affine scales and biases as bf16
    (:73-79,189-195). The 9B decode layer at M = 1 (the headline's shapes) and the 27B
    prefill layer at M = 2048 with bf16 scales and biases, timed as their fp16 entries."""
    import torch

    from raceline_amd.configs import CFG2_9B_STACKED, CFG3_27B, CFG4_PREFILL_M, linear_flops

    out = {}
    L9 = CFG2_9B_STACKED
    l9 = build_layer_copies(L9, copies_for(L9), 1, device, torch.bfloat16)
    r = LayerRunner(l9, L9, 1, device)
    t = time_steps(r, steps, warmup)
    out["layer_9b_m1_bf16"] = {"us_per_step": round(t * 1e6, 2), "GB/s": round(layer_bytes(L9, 1) / t / 1e9, 1)}
    log(f"[bench] 9B layer M=1, bf16 scales: {t * 1e6:.1f} us/step")
    del r, l9
    torch.cuda.empty_cache()
    l27 = build_layer_copies(CFG3_27B, 2, 2, device, torch.bfloat16)
    rp = LayerRunner(l27, CFG3_27B, CFG4_PREFILL_M, device, outliers=0.01)
    tp = time_steps(rp, max(4, steps // 5), 2)
    flops = sum(linear_flops(CFG4_PREFILL_M, K, N) for _, K, N in CFG3_27B)
    out["prefill_27b_m2048_bf16"] = {"us_per_step": round(tp * 1e6, 1), "TFLOP/s": round(flops / tp / 1e12, 1),
                                     "frac_of_mfma_peak": round(flops / tp / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    log(f"[bench] 27B prefill, bf16 scales: {flops / tp / 1e12:.1f} TFLOP/s")
    del rp, l27
    torch.cuda.empty_cache()
    return out


def bench_head(device, steps, warmup):
    """The output head at the reference's vocabulary (src/engine.mm:1634-1638): 248,320 rows
    of hidden 4096 and 5120, affine with bf16 scales (the .rlm format), one token (M = 1)
    and a token with 4 drafts (M = 5), over >= 1 GiB of rotating copies; the largest single
    matrix of a decode pass, HBM-bound like the decode layer."""
    import torch

    from raceline_amd.configs import linear_bytes

    out = {}
    for H in (4096, 5120):
        shapes = [("lm_head", H, HEAD_VOCAB)]
        copies = copies_for(shapes)
        heads = build_layer_copies(shapes, copies, 30 + H, device, torch.bfloat16)
        for M in (1, 5):
            r = LayerRunner(heads, shapes, M, device)
            t = time_steps(r, steps, warmup)
            nb = linear_bytes(M, H, HEAD_VOCAB)
            out[f"head_248k_h{H}_m{M}"] = {"us": round(t * 1e6, 2), "GB/s": round(nb / t / 1e9, 1),
                                           "frac_of_hbm_peak": round(nb / t / 1e9 / HBM_PEAK_GBS, 4),
                                           "algorithmic_bytes": nb}
            log(f"[bench] head 248320 x {H} M={M}: {t * 1e6:.1f} us, {nb / t / 1e9:.0f} GB/s")
            del r
        del heads
        torch.cuda.empty_cache()
    return out


def bench_engine(device, steps, warmup, tmpdir):
    """The engine path over .rlm files (include/rl_engine.h): rl_mlp on a 9B-shaped dense
    layer (post norm, gate_up 4096 -> 2 x 12288 with parts gate and up, SwiGLU, down 12288
    -> 4096 added to h: Engine::encode_mlp, src/engine.mm:943-958) at T = 1 and 5, and on the
    BASELINE MoE layer (router, routing, experts, combine: encode_moe, :965-1059) at T = 1
    and 512, in affine files with bf16 scales written here, one model of enough layers that
    the steps, which rotate over the layers, stream from HBM. Beside each, the sum of its
    parts timed alone the same way: rl_norm, rl_linear on gate_up, the SwiGLU kernel and
    rl_linear on down (ACCUM); or rl_norm, rl_linear on the router and the expert kernels
    (rlq_moe over stacks of the same shapes and scale type packed by the kernel ABI)."""
    import torch

    from raceline_amd import ops, synth
    from raceline_amd.configs import MOE, linear_bytes
    from raceline_amd.model import Engine

    out = {}
    H, I = 4096, 12288
    per_layer = linear_bytes(1, H, 2 * I) + linear_bytes(1, I, H)
    layers = -(-CACHE_DEFEAT_BYTES // per_layer)
    path = os.path.join(tmpdir, "dense_9b_mlp.rlm")
    t0 = time.time()
    synth.write_mlp_model(path, layers, H, I, seed=1)
    log(f"[bench] wrote a {layers}-layer 9B-shaped MLP model ({os.path.getsize(path) / 1e9:.2f} GB) "
        f"in {time.time() - t0:.1f} s")
    with Engine(path, max_chunk=512) as e:
        for T in (1, 5):
            h = synth.random_activations(T, H, 40 + T, device).float()
            xn = torch.empty((T, H), dtype=torch.float16, device=device)
            g = torch.empty((T, 2 * I), dtype=torch.float32, device=device)
            act = torch.empty((T, I), dtype=torch.float16, device=device)

            def swiglu():
                ops.lib.call("rlq_moe_swiglu", g.data_ptr(), g.stride(0), T, I, 0, act.data_ptr(), act.stride(0),
                             ops._stream())

            parts = {
                "rl_mlp": [(lambda i=i: e.mlp(i, h)) for i in range(layers)],
                "norm": [(lambda i=i: lib_norm(e, 1, i, h, xn)) for i in range(layers)],
                "gate_up": [(lambda i=i: e.linear(f"layers.{i}.mlp.gate_up", xn, out=g)) for i in range(layers)],
                "swiglu": [swiglu] * layers,
                "down": [(lambda i=i: e.linear(f"layers.{i}.mlp.down", act, out=h, accum=True)) for i in range(layers)],
            }
            times = {k: time_steps(StepGraphs(v), steps, warmup) for k, v in parts.items()}
            nb = linear_bytes(T, H, 2 * I) + linear_bytes(T, I, H)
            ent = {k + "_us": round(v * 1e6, 2) for k, v in times.items()}
            ent["sum_of_parts_us"] = round(sum(v for k, v in times.items() if k != "rl_mlp") * 1e6, 2)
            ent["GB/s"] = round(nb / times["rl_mlp"] / 1e9, 1)
            out[f"engine_dense_9b_mlp_t{T}"] = ent
            log(f"[bench] engine rl_mlp 9B dense T={T}: {ent['rl_mlp_us']} us (parts {ent['sum_of_parts_us']} us)")
    os.remove(path)

    E, Hm, Im, topk = MOE["E"], MOE["H"], MOE["I"], MOE["topk"]
    per_layer = ops.packed_bytes(Hm, (E + 1) * 2 * Im) + ops.packed_bytes(Im, (E + 1) * Hm)
    layers = max(2, -(-CACHE_DEFEAT_BYTES // per_layer))
    path = os.path.join(tmpdir, "moe_35b.rlm")
    t0 = time.time()
    synth.write_mlp_model(path, layers, Hm, experts=E, topk=topk, moe_inter=Im, seed=2)
    log(f"[bench] wrote a {layers}-layer MoE model ({os.path.getsize(path) / 1e9:.2f} GB) in {time.time() - t0:.1f} s")
    mws = []
    for c in range(layers):
        gu = synth.random_affine((E + 1) * 2 * Im, Hm, 520 + 2 * c, device, packed=False, scale_dtype=torch.bfloat16)
        dn = synth.random_affine((E + 1) * Hm, Im, 521 + 2 * c, device, packed=False, scale_dtype=torch.bfloat16)
        mws.append(ops.pack_moe(gu, dn, E, Hm, Im))
        del gu, dn
    with Engine(path, max_chunk=512) as e:
        for T in MOE["tokens"]:
            # one-token steps draw their own residual rows, so the routing (and the experts
            # read) changes from step to step, as moe_step_logits explains
            n = max(MOE_T1_STEPS, layers) if T == 1 else layers
            hs = [synth.random_activations(T, Hm, 50 + j, device).float() for j in range(n if T == 1 else 1)]
            hs = hs * n if T > 1 else hs
            xn = torch.empty((T, Hm), dtype=torch.float16, device=device)
            lg = torch.empty((T, (E + 1 + 255) // 256 * 256), dtype=torch.float32, device=device)
            logits = moe_step_logits(T, E, layers, device)
            ws = torch.empty(ops.moe_workspace_bytes(T, E, topk, Hm, Im), dtype=torch.uint8, device=device)
            parts = {
                "rl_mlp": [(lambda j=j: e.mlp(j % layers, hs[j])) for j in range(n)],
                "norm": [(lambda j=j: lib_norm(e, 1, j % layers, hs[j], xn)) for j in range(n)],
                "router": [(lambda j=j: e.linear(f"layers.{j % layers}.moe.router", xn, out=lg)) for j in range(n)],
                "experts": [(lambda j=j: ops.moe(xn, logits[j % len(logits)], mws[j % layers], topk, hs[j],
                                                 workspace=ws)) for j in range(n)],
            }
            times = {k: time_steps(StepGraphs(v), steps, warmup) for k, v in parts.items()}
            ent = {k + "_us": round(v * 1e6, 2) for k, v in times.items()}
            ent["sum_of_parts_us"] = round(sum(v for k, v in times.items() if k != "rl_mlp") * 1e6, 2)
            out[f"engine_moe_t{T}"] = ent
            log(f"[bench] engine rl_mlp MoE T={T}: {ent['rl_mlp_us']} us (parts {ent['sum_of_parts_us']} us)")
    del mws
    os.remove(path)
    torch.cuda.empty_cache()
    return out


def lib_norm(e, which, layer, h, xn):
    """rl_norm into a caller's buffer (the engine's Python wrapper allocates its output)."""
    from raceline_amd import lib
    from raceline_amd.model import _check, _stream

    _check(lib.load().rl_norm(e._e, which, layer, h.data_ptr(), h.stride(0), h.shape[0], xn.data_ptr(), xn.stride(0),
                              _stream()), "rl_norm")


def bench_prefill(device, steps, warmup):
    """the 27B layer's four projections at M = 2048 (fp16 activations with
    1% outliers x20), TFLOP/s against the dense fp16 MFMA peak; two weight copies."""
    import torch

    from raceline_amd.configs import CFG3_27B, CFG4_PREFILL_M, linear_flops

    l27 = build_layer_copies(CFG3_27B, 2, 2, device, torch.float16)
    rp = LayerRunner(l27, CFG3_27B, CFG4_PREFILL_M, device, outliers=0.01)
    tp = time_steps(rp, max(4, steps // 5), 2)
    flops = sum(linear_flops(CFG4_PREFILL_M, K, N) for _, K, N in CFG3_27B)
    log(f"[bench] 27B prefill: {flops / tp / 1e12:.1f} TFLOP/s")
    del rp, l27
    torch.cuda.empty_cache()
    ref = dense_fp16_reference(device, CFG3_27B, CFG4_PREFILL_M)
    log(f"[bench] dense fp16 vendor GEMM on the same shapes: {flops / ref / 1e12:.1f} TFLOP/s")
    return {"prefill_27b_m2048": {"us_per_step": round(tp * 1e6, 1), "TFLOP/s": round(flops / tp / 1e12, 1),
                                  "frac_of_mfma_peak": round(flops / tp / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                                  "dense_fp16_vendor_gemm_TFLOP/s": round(flops / ref / 1e12, 1),
                                  "frac_of_dense_fp16_vendor_gemm": round(ref / tp, 3)}}


def dense_fp16_reference(device, shapes, M):
    """Seconds per layer of the vendor GEMM (torch.nn.functional.linear: y = x W^T with W
    [N][K] as the packed weights are) on the same shapes with dense fp16 weights and N(0,1)
    activations: the practical matrix-core ceiling on this box, for comparison only (the
    quantized path never calls it)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(7)
    total = 0.0
    for _, K, N in shapes:
        x = torch.randn((M, K), generator=g, device=device, dtype=torch.float16)
        w = torch.randn((N, K), generator=g, device=device, dtype=torch.float16) * 0.02   # [N][K], as packed
        for _ in range(3):
            torch.nn.functional.linear(x, w)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(10):
            torch.nn.functional.linear(x, w)
        e.record()
        torch.cuda.synchronize()
        total += s.elapsed_time(e) / 10 * 1e-3
        del x, w
    torch.cuda.empty_cache()
    return total


def bench_decode(device, steps, warmup):
    """BASELINE configs 2 and 3: the 9B layer (q/k/v stacked) at M = 1 and 5, the 27B layer at
    M = 1 and 8, each step one pass over rotating weight copies."""
    import torch

    from raceline_amd.configs import CFG2_9B_STACKED, CFG3_27B

    out = {}
    for name, cfg, ms in (("9b", CFG2_9B_STACKED, (1, 5)), ("27b", CFG3_27B, (1, 8))):
        layers = build_layer_copies(cfg, copies_for(cfg), 2, device, torch.float16)
        for M in ms:
            r = LayerRunner(layers, cfg, M, device)
            t = time_steps(r, steps, warmup)
            out[f"layer_{name}_m{M}"] = {"us_per_step": round(t * 1e6, 2),
                                         "GB/s": round(layer_bytes(cfg, M) / t / 1e9, 1)}
            log(f"[bench] {name} layer M={M}: {t * 1e6:.1f} us/step, {layer_bytes(cfg, M) / t / 1e9:.0f} GB/s")
            del r
        del layers
        torch.cuda.empty_cache()
    return out


def bench_launch_cost(device, steps, warmup):
    """The decode kernel's cost per launch at K = 4096 (BASELINE config 1 is N = 4096): the
    average kernel time of back-to-back launches in a captured graph over rotating weight
    copies (>= 1 GiB, so every launch streams from HBM) for N = 512 ... 49152, and the
    straight line t = t0 + bytes / rate fitted to the N >= 4096 points by least squares:
    t0 is what a launch costs beyond streaming its bytes (dispatch, the first loads'
    latency, the last wave's reduction and stores). Also the time of a launch that does
    next to nothing (torch's fill of one float) in the same kind of graph."""
    import torch

    from raceline_amd import synth
    from raceline_amd.configs import linear_bytes

    K = 4096
    rows = []
    for N in (512, 1024, 2048, 4096, 8192, 16384, 24576, 49152):
        per = linear_bytes(1, K, N)
        copies = max(2, min(512, -(-CACHE_DEFEAT_BYTES // per)))
        shapes = [("w", K, N)]
        layers = [[synth.random_affine(N, K, 7 + c, device)] for c in range(copies)]
        launches = max(copies, 64)
        t = time_kernel(layers, shapes, 1, 0, device, launches=launches)
        rows.append((N, per, t))
        log(f"[bench] decode launch K={K} N={N}: {t * 1e6:.2f} us, {per / t / 1e9:.0f} GB/s ({copies} copies)")
        del layers
        torch.cuda.empty_cache()
    fit = [(b, t) for N, b, t in rows if N >= 4096]
    n = len(fit)
    mb = sum(b for b, _ in fit) / n
    mt = sum(t for _, t in fit) / n
    slope = sum((b - mb) * (t - mt) for b, t in fit) / sum((b - mb) ** 2 for b, _ in fit)
    t0 = mt - slope * mb
    # a launch of almost no work, in a graph of back-to-back launches on one stream
    one = torch.zeros(1, device=device)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(256):
            one.fill_(1.0)
    t_empty = timed_replay(g, stream) / 256
    log(f"[bench] fit over N >= 4096: t0 = {t0 * 1e6:.2f} us per launch, stream rate {1 / slope / 1e9:.0f} GB/s; "
        f"fill of one float: {t_empty * 1e6:.2f} us per launch")
    return {"K": K, "points": [{"N": N, "bytes": b, "us": round(t * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
                               for N, b, t in rows],
            "fit_t0_us": round(t0 * 1e6, 2), "fit_stream_GBps": round(1 / slope / 1e9, 1),
            "empty_launch_us": round(t_empty * 1e6, 2)}


def bench_stream_probe(device, reps=8):
    """What this box's HBM delivers to plain streaming kernels, as context for the roofline
    fractions (which stay against 8 TB/s): a read stream (rlq_stream_read: 16-byte
    non-temporal loads from every CU over 1 GiB, nothing written) and a copy stream
    (torch.neg from one 1 GiB tensor into another), each `reps` times back to back in a
    captured graph over two pairs of buffers (4 GiB in all, far past the 256 MB Infinity
    Cache), replayed between two events."""
    import torch

    from raceline_amd import ops

    n = 1 << 28                       # 1 GiB of fp32
    bufs = [torch.ones(n, dtype=torch.float32, device=device) for _ in range(4)]
    out = torch.zeros(1, dtype=torch.float32, device=device)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()

    def timed(fn, reps=reps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            for i in range(2):
                fn(i)                 # eager warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for i in range(reps):
                fn(i)
        return timed_replay(g, stream) / reps

    t_read = timed(lambda i: ops.lib.call("rlq_stream_read", bufs[i % 2].data_ptr(), 4 * n, out.data_ptr(),
                                          ops._stream()))
    t_copy = timed(lambda i: torch.neg(bufs[i % 2], out=bufs[2 + i % 2]))
    # the same read stream at the headline kernel's size (the 9B gate_up's algorithmic bytes
    # at M = 1), each launch on the next slice of the 4 GiB, as the decode launches rotate
    small = 56729600 // 256 * 256
    slices = [(b, o) for b in range(4) for o in range(0, 4 * n - small + 1, small)]
    t_small = timed(lambda i: ops.lib.call("rlq_stream_read", bufs[slices[i % len(slices)][0]].data_ptr() +
                                           slices[i % len(slices)][1], small, out.data_ptr(), ops._stream()),
                    reps=len(slices))
    res = {"read_GBps": round(4 * n / t_read / 1e9, 1), "copy_GBps": round(8 * n / t_copy / 1e9, 1),
           "bytes_read": 4 * n, "read_56.7MB_us": round(t_small * 1e6, 2),
           "read_56.7MB_GBps": round(small / t_small / 1e9, 1),
           "kernels": "rlq_stream_read (read) and torch.neg (copy) of 1 GiB, and rlq_stream_read of 56.7 MB "
                      "slices of 4 GiB, graph-timed"}
    log(f"[bench] HBM stream probe: read {res['read_GBps']} GB/s, copy {res['copy_GBps']} GB/s, "
        f"56.7 MB reads {res['read_56.7MB_us']} us each ({res['read_56.7MB_GBps']} GB/s)")
    del bufs
    torch.cuda.empty_cache()
    return res


def bench_part(part, steps, warmup):
    import torch

    from raceline_amd import lib

    lib.load()
    dev = torch.device("cuda:0")
    log(f"[bench] part {part}")
    if part == "engine":
        import tempfile

        with tempfile.TemporaryDirectory() as tmp:
            return bench_engine(dev, steps, warmup, tmp)
    if part == "stream":
        return bench_stream_probe(dev)
    fn = {"prefill": bench_prefill, "moe": bench_moe, "decode": bench_decode, "epilogue": bench_native_epilogue,
          "launch": bench_launch_cost, "bf16": bench_bf16, "head": bench_head}[part]
    return fn(dev, steps, warmup)


def time_kernel(layers, shapes, M, idx, device, launches, kernel=0, outliers=0.0):
    """Average duration of projection idx's kernel: a captured graph of `launches`
    back-to-back launches over the rotating copies, replayed between two events on the
    stream the kernels run on."""
    import torch

    from raceline_amd import ops, synth

    _, K, N = shapes[idx]
    x = synth.random_activations(M, K, 99, device, outliers)
    y = torch.empty((M, N), dtype=torch.float32, device=device)
    ops._WS.get(device, ops.workspace_bytes(M, K, N))
    torch.cuda.synchronize()          # x, y and the workspace are ready before the side stream uses them
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for c in range(len(layers)):
            ops.linear(x, layers[c][idx], out=y, kernel=kernel)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(launches):
            ops.linear(x, layers[i % len(layers)][idx], out=y, kernel=kernel)
    return timed_replay(g, stream) / launches


def cpu_model() -> str:
    """The host CPU's model name (what lscpu reports), from /proc/cpuinfo."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        return int(max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1]))
    except Exception:  # noqa: BLE001
        return int(os.environ.get("OPENBLAS_NUM_THREADS", os.cpu_count() or 1))


def _median(v):
    v = sorted(v)
    return v[len(v) // 2]


def _host_affine(device, K, N, seed):
    import numpy as np
    import torch

    from raceline_amd import synth

    w, s, b = synth.random_affine(N, K, seed, device, packed=False)
    return (w.cpu().numpy().view(np.uint32), s.cpu().view(torch.int16).numpy().view(np.uint16),
            b.cpu().view(torch.int16).numpy().view(np.uint16))


def _cpu_linear(mats, xs, runs):
    """The reference's CPU path over a list of matrices (numpy unpack + dequant, then the
    fp32 BLAS matmul): one warm-up, then the median of `runs` of each phase, in ms."""
    import numpy as np

    import oracle as O

    deq, mm = [], []
    for r in range(runs + 1):
        td = tm = 0.0
        for (w, s, b), x in zip(mats, xs):
            a = time.perf_counter()
            W = O.dequant_affine(O.unpack_nibbles_u32(w), s, b, "f16")
            m = time.perf_counter()
            _ = x.astype(np.float32) @ W.T
            e = time.perf_counter()
            td += m - a
            tm += e - m
        if r:   # the first pass warms up
            deq.append(td)
            mm.append(tm)
    return _median(deq) * 1e3, _median(mm) * 1e3


def cpu_baseline(device):
    """The reference's CPU path (numpy dequant + fp32 BLAS matmul, the oracle's restatement
    of tools/convert.py:82-89 and kernels/linear.metal:4) on every BASELINE config, on this
    host: dequant (single-threaded numpy) and matmul (multi-threaded BLAS) timed apart, the
    median of several runs after a warm-up (bounded samples where a config is large, as
    each entry says). The headline entry is config 2's layer at M = 1 (q/k/v stacked)."""
    import numpy as np
    import torch

    from raceline_amd import synth
    from raceline_amd.configs import CFG1_SINGLE, CFG2_9B_STACKED, CFG3_27B, CFG4_PREFILL_M, MOE, linear_bytes

    threads, model = blas_threads(), cpu_model()
    table = {}

    def layer(name, shapes, Ms, runs, seed):
        mats = [_host_affine(device, K, N, seed + i) for i, (_, K, N) in enumerate(shapes)]
        for M in Ms:
            xs = [synth.random_activations(M, K, seed + 50 + i, device, 0.01 if M > 8 else 0.0).cpu().numpy()
                  for i, (_, K, _) in enumerate(shapes)]
            d, m = _cpu_linear(mats, xs, runs)
            nbytes = sum(linear_bytes(M, K, N) for _, K, N in shapes)
            flops = sum(2 * M * K * N for _, K, N in shapes)
            table[f"{name}_m{M}"] = {"dequant_ms": round(d, 2), "matmul_ms": round(m, 2), "total_ms": round(d + m, 2),
                                     "GB/s": round(nbytes / (d + m) / 1e6, 3),
                                     "TFLOP/s": round(flops / (d + m) / 1e9, 4), "runs": runs}
            log(f"[bench] CPU {name} M={M}: dequant {d:.1f} ms + matmul {m:.1f} ms")
        del mats

    layer("cfg1_single", CFG1_SINGLE, (1,), 5, 4200)
    layer("cfg2_9b_layer", CFG2_9B_STACKED, (1, 5), 5, 4242)
    layer("cfg3_27b_layer", CFG3_27B, (1, 8), 3, 4300)
    layer("cfg4_27b_prefill", CFG3_27B, (CFG4_PREFILL_M,), 2, 4300)
    # config 5: the MoE layer restated on the host (route, then each expert's dequant and its
    # rows' gate/up, SwiGLU, down), at T = 1 and, for T = 512, a sample of 32 of the experts
    # with their routed rows, scaled to all of them
    E, H, I, topk = MOE["E"], MOE["H"], MOE["I"], MOE["topk"]
    gu = _host_affine(device, H, (E + 1) * 2 * I, 4400)
    dn = _host_affine(device, I, (E + 1) * H, 4401)
    import oracle as O
    for T in MOE["tokens"]:
        x = synth.random_activations(T, H, 4402 + T, device).cpu().numpy()
        g = torch.Generator(device=device)
        g.manual_seed(4403 + T)
        logits = torch.randn((T, E + 1), generator=g, device=device, dtype=torch.float32).cpu().numpy()
        sel, _ = O.moe_route(logits, E, topk)
        experts = sorted(set(int(e) for e in sel))
        sample = experts if T == 1 else experts[:: max(1, len(experts) // 32)][:32]
        rows_of = {e: [a // (topk + 1) for a in range(len(sel)) if int(sel[a]) == e] for e in sample}
        deq, mm = [], []
        for r in range(4):
            td = tm = 0.0
            for e in sample:
                a = time.perf_counter()
                rg, rd = slice(e * 2 * I, (e + 1) * 2 * I), slice(e * H, (e + 1) * H)
                Wg = O.dequant_affine(O.unpack_nibbles_u32(gu[0][rg]), gu[1][rg], gu[2][rg], "f16")
                Wd = O.dequant_affine(O.unpack_nibbles_u32(dn[0][rd]), dn[1][rd], dn[2][rd], "f16")
                m = time.perf_counter()
                gg = x[rows_of[e]].astype(np.float32) @ Wg.T
                act = (gg[:, :I] / (1 + np.exp(-gg[:, :I])) * gg[:, I:]).astype(np.float16)
                _ = act.astype(np.float32) @ Wd.T
                f = time.perf_counter()
                td += m - a
                tm += f - m
            if r:
                deq.append(td * len(experts) / len(sample))
                mm.append(tm * len(experts) / len(sample))
        d, m = _median(deq) * 1e3, _median(mm) * 1e3
        table[f"cfg5_moe_t{T}"] = {"dequant_ms": round(d, 2), "matmul_ms": round(m, 2), "total_ms": round(d + m, 2),
                                   "experts": len(experts), "experts_timed": len(sample), "runs": 3}
        log(f"[bench] CPU MoE T={T}: dequant {d:.1f} ms + matmul {m:.1f} ms ({len(sample)} of {len(experts)} experts)")
    del gu, dn
    head = table["cfg2_9b_layer_m1"]
    return {
        "value": head["GB/s"], "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"config 2 layer (q/k/v stacked, o, gate_up, down) at M=1: numpy unpack+dequant (1 thread) "
                   f"{head['dequant_ms']} ms + fp32 BLAS matmul ({threads} threads) {head['matmul_ms']} ms, "
                   f"median of {head['runs']} after a warm-up; host: {model}, {os.cpu_count()} logical CPUs; "
                   f"every config under detail.cpu_baseline_per_config"),
        "cpu_model": model, "per_config": table,
    }


PROFILE_TRAFFIC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "gemv_q4a_9b_gate_up_m1_traffic.txt")
CALIBRATION_BYTES = 256 << 20  # the elementwise calibration kernel reads and writes this much


def profile_dominant(launches):
    """--profile: the dominant kernel alone (9B gate_up at M=1), launched eagerly over its
    rotating weight copies, then a plain elementwise kernel of known traffic (torch.neg
    over 256 MiB of float32: reads 256 MiB, writes 256 MiB) that calibrates rocprofv3's
    FETCH_SIZE and WRITE_SIZE counters. Meant to run under rocprofv3."""
    import torch

    from raceline_amd import lib, ops, synth
    from raceline_amd.configs import CFG2_9B

    lib.load()
    dev = torch.device("cuda:0")
    _, K, N = [c for c in CFG2_9B if c[0] == "gate_up"][0]
    shapes = [("gate_up", K, N)]
    copies = copies_for(shapes)
    ws = [synth.random_affine(N, K, 1 + 1000 * c, dev) for c in range(copies)]
    x = synth.random_activations(1, K, 99, dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    for i in range(launches):
        ops.linear(x, ws[i % copies], out=y)
    torch.cuda.synchronize()
    a = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(10):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    log(f"[profile] gemv_q4a K={K} N={N} M=1: {launches} launches over {copies} copies; "
        f"calibration: 10 x torch.neg over {CALIBRATION_BYTES >> 20} MiB")


def profile_gemv8(launches):
    """--profile gemv8: the 27B gate_up (K = 5120, N = 34816) at M = 1 and at M = 8 (the MTP
    draft regime), launched eagerly in turn over rotating weight copies (the one-tile kernel
    at M = 1, the two-tile kernel with rows staged in LDS at M = 8), then the calibration
    kernel of profile_dominant. Meant to run under rocprofv3 --pmc: the two kernels' counters
    compare the same weights' traffic at one and eight tokens."""
    import torch

    from raceline_amd import lib, ops, synth
    from raceline_amd.configs import CFG3_27B

    lib.load()
    dev = torch.device("cuda:0")
    _, K, N = [c for c in CFG3_27B if c[0] == "gate_up"][0]
    copies = copies_for([("gate_up", K, N)])
    ws = [synth.random_affine(N, K, 5 + 1000 * c, dev) for c in range(copies)]
    xs = {M: synth.random_activations(M, K, 90 + M, dev) for M in (1, 8)}
    ys = {M: torch.empty((M, N), dtype=torch.float32, device=dev) for M in (1, 8)}
    for M in (1, 8):
        ops._WS.get(dev, ops.workspace_bytes(M, K, N))
    for i in range(launches):
        for M in (1, 8):
            ops.linear(xs[M], ws[i % copies], out=ys[M])
    torch.cuda.synchronize()
    a = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(10):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    log(f"[profile] gemv_q4a K={K} N={N} M=1 and M=8: {launches} launches each over {copies} copies; "
        f"calibration: 10 x torch.neg over {CALIBRATION_BYTES >> 20} MiB")


def profile_moe(launches, T=512):
    """--profile moe: the MoE layer (H=2048, E=256 + shared, I=512, top-8) at T tokens,
    launched eagerly over rotating copies of the experts (each step routes, multiplies and
    combines: moe_topk, moe_sort, the gate/up and down expert kernels, moe_combine), then
    the calibration kernel of profile_dominant. Meant to run under rocprofv3 --pmc."""
    import torch

    from raceline_amd import lib, ops, synth
    from raceline_amd.configs import MOE

    lib.load()
    dev = torch.device("cuda:0")
    E, H, I, topk = MOE["E"], MOE["H"], MOE["I"], MOE["topk"]
    per_copy = ops.packed_bytes(H, (E + 1) * 2 * I) + ops.packed_bytes(I, (E + 1) * H)
    copies = max(2, -(-CACHE_DEFEAT_BYTES // per_copy))
    mws = []
    for c in range(copies):
        gu = synth.random_affine((E + 1) * 2 * I, H, 500 + 2 * c, dev, packed=False)
        dn = synth.random_affine((E + 1) * H, I, 501 + 2 * c, dev, packed=False)
        mws.append(ops.pack_moe(gu, dn, E, H, I))
        del gu, dn
    x = synth.random_activations(T, H, 600 + T, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(601 + T)
    logits = torch.randn((T, E + 1), generator=g, device=dev, dtype=torch.float32)
    h = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ws = torch.empty(ops.moe_workspace_bytes(T, E, topk, H, I), dtype=torch.uint8, device=dev)
    for i in range(launches):
        ops.moe(x, logits, mws[i % copies], topk, h, workspace=ws)
    torch.cuda.synchronize()
    distinct = int(torch.unique(ops.moe_route(logits, E, topk).sel).numel())
    a = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(10):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    log(f"[profile] MoE T={T}: {launches} layer steps over {copies} copies of {per_copy / 1e6:.1f} MB, "
        f"{distinct} distinct experts; calibration: 10 x torch.neg over {CALIBRATION_BYTES >> 20} MiB")


def profile_gemm(launches):
    """--profile gemm: the prefill kernel alone on the 27B gate_up (M = 2048, K = 5120,
    N = 34816, activations with 1% outliers x20), launched eagerly over two weight copies,
    then the calibration kernel of profile_dominant. Meant to run under rocprofv3 --pmc."""
    import torch

    from raceline_amd import lib, ops, synth
    from raceline_amd.configs import CFG3_27B, CFG4_PREFILL_M

    lib.load()
    dev = torch.device("cuda:0")
    _, K, N = [c for c in CFG3_27B if c[0] == "gate_up"][0]
    M = CFG4_PREFILL_M
    ws = [synth.random_affine(N, K, 1 + 1000 * c, dev) for c in range(2)]
    x = synth.random_activations(M, K, 99, dev, 0.01)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    for i in range(launches):
        ops.linear(x, ws[i % 2], out=y)
    torch.cuda.synchronize()
    a = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(10):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    log(f"[profile] gemm4 M={M} K={K} N={N}: {launches} launches over 2 copies; "
        f"calibration: 10 x torch.neg over {CALIBRATION_BYTES >> 20} MiB")


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the calibration kernel), or None."""
    try:
        for line in open(PROFILE_TRAFFIC):
            if line.startswith("traffic_bytes_per_launch"):
                return int(float(line.split("=")[1]))
    except (OSError, ValueError, IndexError):
        pass
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline only (no detail configs, no CPU baseline)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--part", choices=["prefill", "moe", "decode", "epilogue", "launch", "bf16", "head", "engine",
                                       "stream", "cpu"],
                    help="run only this part of the detail (for rocprofv3); prints its figures as JSON")
    ap.add_argument("--profile", nargs="?", const="gemv", choices=["gemv", "gemv8", "moe", "gemm"],
                    help="launch only the dominant kernel (gemv), the 27B gate_up at M=1 and M=8 (gemv8), the MoE "
                         "layer at T=512 (moe) or the prefill kernel on the 27B gate_up (gemm), eagerly, and a "
                         "calibration kernel (for rocprofv3 --pmc)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build's path runs on a single MI355X (the multi-GPU "
              "sharding is a design only); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.profile == "gemv":
        profile_dominant(max(args.steps, 40))
        return
    if args.profile == "gemv8":
        profile_gemv8(max(args.steps, 20))
        return
    if args.profile == "moe":
        profile_moe(max(args.steps, 20))
        return
    if args.profile == "gemm":
        profile_gemm(max(min(args.steps, 20), 6))
        return
    if args.part == "cpu":
        import torch

        print(json.dumps(cpu_baseline(torch.device("cuda:0"))), flush=True)
        return
    if args.part:
        print(json.dumps(bench_part(args.part, args.steps, args.warmup)), flush=True)
        return

    import torch

    from raceline_amd import lib
    from raceline_amd.configs import CFG2_9B, CFG2_9B_STACKED, CFG3_27B, linear_bytes

    lib.load()
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    sd = torch.float16

    # ---------------- headline: 9B decode layer (q/k/v stacked), M = 1
    L9 = CFG2_9B_STACKED
    copies = copies_for(L9)
    log(f"[bench] building {copies} copies of the 9B layer ({layer_bytes(L9, 1) / 1e6:.1f} MB each)")
    l9 = build_layer_copies(L9, copies, 1, dev, sd)
    run1 = LayerRunner(l9, L9, 1, dev)
    t1 = time_steps(run1, args.steps, args.warmup)
    bytes1 = layer_bytes(L9, 1)
    value = bytes1 / t1 / 1e9
    log(f"[bench] 9B layer M=1: {t1 * 1e6:.1f} us/step, {value:.0f} GB/s")

    # dominant kernel: gate_up GEMV at M=1
    gu = [i for i, (n, _, _) in enumerate(L9) if n == "gate_up"][0]
    _, Kg, Ng = L9[gu]
    t_gu = time_kernel(l9, L9, 1, gu, dev, launches=4 * copies)
    ach = linear_bytes(1, Kg, Ng) / t_gu / 1e9
    roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                "kernel": "gemv_q4a_kernel<1,8,0,false,0> (9B gate_up, M=1, K=4096, N=24576)",
                "avg_launch_us": round(t_gu * 1e6, 2), "algorithmic_bytes": linear_bytes(1, Kg, Ng)}

    detail = {"layer_9b_m1": {"us_per_step": round(t1 * 1e6, 2), "GB/s": round(value, 1)}}
    if not args.quick:
        per = {}
        for i, (name, K, N) in enumerate(L9):
            t = time_kernel(l9, L9, 1, i, dev, launches=2 * copies)
            per[name] = {"us": round(t * 1e6, 2), "GB/s": round(linear_bytes(1, K, N) / t / 1e9, 1)}
        detail["proj_9b_m1"] = per
        run5 = LayerRunner(l9, L9, 5, dev)
        t5 = time_steps(run5, args.steps, args.warmup)
        detail["layer_9b_m5"] = {"us_per_step": round(t5 * 1e6, 2),
                                 "GB/s": round(layer_bytes(L9, 5) / t5 / 1e9, 1)}
        del run1, run5, l9
        torch.cuda.empty_cache()
        # the same layer with q, k and v as three matrices (six launches)
        c6 = copies_for(CFG2_9B)
        l6 = build_layer_copies(CFG2_9B, c6, 1, dev, sd)
        r6 = LayerRunner(l6, CFG2_9B, 1, dev)
        t6 = time_steps(r6, args.steps, args.warmup)
        detail["layer_9b_m1_six_launches"] = {"us_per_step": round(t6 * 1e6, 2),
                                              "GB/s": round(layer_bytes(CFG2_9B, 1) / t6 / 1e9, 1)}
        del r6, l6
        torch.cuda.empty_cache()
        detail["hbm_stream_probe"] = bench_stream_probe(dev)

        c27 = copies_for(CFG3_27B)
        log(f"[bench] building {c27} copies of the 27B layer")
        l27 = build_layer_copies(CFG3_27B, c27, 2, dev, sd)
        for M in (1, 8):
            r = LayerRunner(l27, CFG3_27B, M, dev)
            t = time_steps(r, args.steps, args.warmup)
            detail[f"layer_27b_m{M}"] = {"us_per_step": round(t * 1e6, 2),
                                         "GB/s": round(layer_bytes(CFG3_27B, M) / t / 1e9, 1)}
            del r
        del l27
        torch.cuda.empty_cache()
        # prefill: M = 2048, compute bound; two copies are plenty
        detail.update(bench_prefill(dev, args.steps, args.warmup))
        detail.update(bench_moe(dev, args.steps, args.warmup))
        detail.update(bench_native_epilogue(dev, args.steps, args.warmup))
        detail.update(bench_bf16(dev, args.steps, args.warmup))
        detail.update(bench_head(dev, args.steps, args.warmup))
        import tempfile

        with tempfile.TemporaryDirectory() as tmp:
            detail.update(bench_engine(dev, args.steps, args.warmup, tmp))

    cpu = None
    if not args.quick and not args.no_cpu:
        log("[bench] CPU baseline (numpy dequant + BLAS matmul)")
        cpu = cpu_baseline(dev)

    line = {
        "metric": "4-bit GEMV achieved HBM GB/s at M=1 (9B decode layer, 6 projections, q/k/v stacked)",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(t1 * 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (seeded N(0,0.02) weights quantized on device, fp16 N(0,1) activations)",
        "config": {"workload": "9B-class decode layer projections q,k,v (one stacked matrix, as the "
                               "reference's attn.qkv),o,gate_up,down; 4-bit affine g64, "
                               "fp16 scales+biases, M=1, fp32 accumulate", "global_batch": 1, "seq_len": 1,
                   "parallelism": "single GPU", "weight_copies": copies, "bytes_per_step": bytes1},
        "roofline": roofline,
        "cpu_baseline": None if cpu is None else {k: v for k, v in cpu.items() if k != "per_config"},
        "detail": detail,
    }
    if cpu is not None:
        line["cpu_baseline"]["value"] = round(cpu["value"], 3)
        detail["cpu_baseline_per_config"] = cpu["per_config"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
