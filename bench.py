#!/usr/bin/env python3
"""Benchmark of the full-attention hot path on one MI355X (gfx950).

Headline (BASELINE.json metric): decode attention KV GB/s at 32K context, Qwen3-Next shape
(16 Q / 2 KV heads, head_dim 256, partial RoPE 64, theta 1e7), batch 1. One step = the whole attention
body between the projections for one full-attention layer — fused QK-norm + RoPE + fp16 KV append,
split-KV attend, LSE combine with the sigmoid gate — i.e. the three dispatches of the reference's
Qwen4Vulkan::attention (src/qwen4_vk.cpp:968-992). Bytes are the algorithmic K/V bytes: every fp16 cache
row read once, 2 * rows * NKV * D * 2.

The timed steps rotate over `--slots` distinct layer caches (1 GiB at 32K) so that the 256 MB
Infinity Cache cannot serve them: HBM is measured, not cache. Inputs are synthetic (seeded N(0,1)),
already resident in HBM when the timed region starts.

The same JSON line carries the other BASELINE configurations (16K decode with the reference's 64
splits, the 4-token MTP verify at 32K, 256K decode with 1% of keys x8, and the 2,048-token causal
prefill on 2,048 cached tokens in TFLOP/s), the roofline of the dominant kernel (its mean launch
duration from HIP events around batches of 16 back-to-back launches on the stream the kernels run on;
HBM traffic per launch from the committed rocprofv3 PMC summary in profiles/), and the CPU baseline:
the reference's CPU attention timed on this host's cores over a bounded sample.

Two QSA workloads (the block-sparse path past the indexer's budget, src/qwen4_vk.cpp:942-984) time the whole
layer step on the GPU at 32K: pool the new indexer key, select the token's blocks (4 indexer heads of 128
dims, a budget of 2,048 keys, blocks of 4 or 64 keys), and the one-launch decode over the tiles the
selection leaves visible; their bytes are the K/V bytes of the visible keys. QSA at 256K runs against the
dense 256K step.

Two projection workloads (proj_q8_n1, proj_q8_n4) time the layer's four projections around the attention
(Qwen4Vulkan::mat on planar Q8_0 weights: query + gate, key, value, output at hidden 2,048) for one decode
token and a 4-token verify pass (query + gate, key and value in one qwattn_mat_multi call, which shares the
layer input, then the output projection); their bytes are the weights, read once a step. A third (proj_q8_n2048) runs
them over a 2,048-token prefill chunk on the tiled MFMA GEMM and reports TFLOP/s (2 n rows cols a projection).
layer_32k_q8 times a whole full-attention layer at decode (32,768 cached + 1): the query + gate, key and value
projections, the attention layer body and the output projection; its bytes are the K/V rows and the weights.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12         # B/s, MI355X HBM3E
MFMA_F16_PEAK = 2.5e15    # FLOP/s, dense fp16/bf16 MFMA
NH, NKV, D, R, THETA, EPS = 16, 2, 256, 64, 1e7, 1e-6


def kv_bytes(rows):
    return 2 * rows * NKV * D * 2


def causal_flops(pos, n):
    return 4 * D * NH * (n * pos + n * (n + 1) // 2)


def load_package():
    import importlib.util
    pkg = os.path.join(ROOT, "qwen3-local-test_amd")
    if "qwattn_amd" in sys.modules:
        return sys.modules["qwattn_amd"]
    spec = importlib.util.spec_from_file_location("qwattn_amd", os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qwattn_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


class Workload:
    """Device state of one configuration: a context with `slots` layer caches filled with seeded N(0,1)
    fp16 rows, and the projection outputs of the n new tokens."""

    def __init__(self, qw, name, pos, n, slots, n_split=0, in_dtype="f32", heavy_frac=0.0, seed=0):
        import torch
        self.name, self.pos, self.n, self.slots, self.n_split = name, pos, n, slots, n_split
        rows = pos + n
        self.cap = (rows + 31) // 32 * 32
        self.att = qw.Attention(NH, NKV, D, R, THETA, EPS, max_ctx=self.cap, max_tokens=max(n, 1),
                                max_splits=1024)
        self.att.kv_alloc(slots, self.cap)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.slot_views = []
        for s in range(slots):
            kc, vc, cap = self.att.kv_slot(s)
            kc.normal_(generator=g)
            vc.normal_(generator=g)
            if heavy_frac > 0:  # post-norm cache rows scaled x8 (softmax-range stress)
                krows = qw.k_rows(kc, cap, NKV, D)
                idx = torch.randperm(rows, device="cuda", generator=g)[:max(1, int(rows * heavy_frac))]
                krows[idx] *= 8.0
                kc.copy_(qw.k_block(krows))
                del krows
            self.slot_views.append((kc, vc, cap))
        dt = torch.float32 if in_dtype == "f32" else torch.bfloat16
        self.qg = torch.randn((n, NH, 2 * D), device="cuda", generator=g).to(dt)
        self.k = torch.randn((n, NKV, D), device="cuda", generator=g).to(dt)
        self.v = torch.randn((n, NKV, D), device="cuda", generator=g).to(dt)
        self.qn = 0.1 * torch.randn(D, device="cuda", generator=g)
        self.kn = 0.1 * torch.randn(D, device="cuda", generator=g)
        self.split = n * (NH // NKV) <= 32 and n <= 8
        # decode and verify: the combine runs inside the attend launch, on the last chunks of each KV head
        # (up to 8 query rows) or 16-row slice, when each has at least as many chunks as rows (the
        # automatic split count gives 128 at 32K for decode, 64 for the verify's slices)
        rows = n * (NH // NKV)
        self.one_launch = self.split and (n_split == 0 or n_split >= min(rows, 16))
        # prefill: the kernel normalizes the query rows itself (the layer entry point's path for this
        # rope width), so no query buffer
        self.q = None
        self.out = torch.zeros((n, NH, D), device="cuda")
        self.rope = self.att.rope_table()
        self.used = None

    def step(self, slot):
        """One attention layer body on layer cache `slot` through the layer entry point."""
        self.att.layer_attention(slot, self.qg, self.k, self.v, self.qn, self.kn, self.out, self.pos, self.n,
                                 self.n_split)

    def step_events(self, slot, ev):
        """The same kernels through the per-dispatch entry points, with HIP events around each kernel."""
        a = self.att
        kc, vc, cap = self.slot_views[slot]
        ev[0].record()
        if self.one_launch:
            self.used = a.decode(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, self.out, self.pos,
                                 self.n, self.n_split)
            ev[1].record()
        elif self.split:
            self.used = a.decode_partial(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, self.pos,
                                         self.n, self.n_split)
            ev[1].record()
            a.combine(self.qg, self.out, self.n, self.used)
        else:
            a.qk_norm_rope_append(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, None,
                                  self.pos, self.n)
            ev[1].record()
            a.attend_prefill_qg(self.qg, self.qn, self.rope, kc, vc, cap, self.out, self.pos, self.n)
        ev[2].record()

    def main_only(self, slot):
        """The dominant kernel alone (it is idempotent: the fused decode rewrites the same new rows, the
        prefill reads the projection output and the rows the last K/V append left)."""
        a = self.att
        kc, vc, cap = self.slot_views[slot]
        if self.one_launch:
            a.decode(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, self.out, self.pos, self.n,
                     self.n_split)
        elif self.split:
            a.decode_partial(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, self.pos, self.n,
                             self.n_split)
        else:
            a.attend_prefill_qg(self.qg, self.qn, self.rope, kc, vc, cap, self.out, self.pos, self.n)

    def close(self):
        self.slot_views = []
        self.att.close()


class QsaWorkload(Workload):
    """A QSA layer step past the budget (the reference's masked path, src/qwen4_vk.cpp:942-984), all on the
    GPU: pool the new token's indexer key, select its blocks, then the one-launch decode over the keys the
    selection leaves visible. Indexer: IH heads of ID dims, blocks of CR keys, a budget of BUDGET keys;
    every layer slot has its own raw and pooled key arrays, built once over the cached history."""
    IH, ID, BUDGET = 4, 128, 2048

    def __init__(self, qw, name, pos, n, slots, cr, seed=0):
        import torch
        self.CR = cr
        super().__init__(qw, name, pos, n, slots, 0, "f32", 0.0, seed)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + 1000)
        self.qsa = True
        self.raw, self.pooled = [], []
        self.ik = torch.randn((n, self.ID), device="cuda", generator=g)
        self.iq = torch.randn((n, self.IH, self.ID), device="cuda", generator=g)
        self.kg = 1 + 0.1 * torch.randn(self.ID, device="cuda", generator=g)
        self.qgam = 1 + 0.1 * torch.randn(self.ID, device="cuda", generator=g)
        for s in range(slots):
            raw = torch.zeros((self.cap, self.ID), device="cuda")
            pooled = torch.zeros((self.cap // self.CR + 1, self.ID), device="cuda")
            hist = torch.randn((pos, self.ID), device="cuda", generator=g)
            self.att.qsa_pool(hist, self.kg, self.CR, raw, pooled, self.cap, 0, pos)
            del hist
            self.raw.append(raw)
            self.pooled.append(pooled)
        self.kbits = torch.zeros((n, (pos + n + 31) // 32), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()

    def select(self, slot):
        # pool + select in one call: at this position no block completes, so one launch
        self.att.qsa_index(self.ik, self.iq, self.kg, self.qgam, self.CR, self.BUDGET, self.raw[slot],
                           self.pooled[slot], self.cap, self.pos, self.n, None, self.kbits)

    def step(self, slot):
        self.select(slot)
        self.att.layer_attention_qsa(slot, self.qg, self.k, self.v, self.qn, self.kn, self.out, self.pos, self.n,
                                     self.kbits)

    def step_events(self, slot, ev):
        kc, vc, cap = self.slot_views[slot]
        ev[0].record()
        self.select(slot)
        ev[1].record()
        self.used = self.att.decode_qsa(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, self.out,
                                        self.pos, self.n, 0, self.kbits)
        ev[2].record()

    def main_only(self, slot):
        kc, vc, cap = self.slot_views[slot]
        self.att.decode_qsa(self.qg, self.k, self.v, self.qn, self.kn, self.rope, kc, vc, cap, self.out, self.pos,
                            self.n, 0, self.kbits)

    def visible(self):
        """(visible keys, keys of the 32-key tiles that hold one) of the last selection."""
        import numpy as np
        w = self.kbits[0].cpu().numpy().view(np.uint32)
        rows = self.pos + self.n
        bits = np.unpackbits(w.view(np.uint8), bitorder="little")  # bit j of word i: key 32 i + j
        bits[rows:] = 0
        return int(bits.sum()), int(bits.reshape(-1, 32).any(axis=1).sum()) * 32

    def close(self):
        self.raw, self.pooled = [], []
        super().close()


_SLEEP_PER_MS = None
KERNEL_BATCHES = 50  # batches of 16 launches timed for the dominant kernel's duration (median reported)


class MatWorkload:
    """The attention layer's four projections (Qwen4Vulkan::mat, src/qwen4_vk.cpp:848-856, on the q4_matmul_q8
    pipeline) for n tokens at hidden 2,048: query + gate (8,192 x 2,048), key and value (512 x 2,048 each) and
    output (2,048 x 4,096), planar Q8_0 weights (seeded int8, scales 0.02 x U(0.5, 1.5)); every layer slot has
    its own weights (30.7 MB a slot), rotated like the K/V caches. Bytes: the weights read once (one byte per
    weight plus a float scale per 32)."""
    HIDDEN = 2048
    SHAPES = [(NH * 2 * D, HIDDEN), (NKV * D, HIDDEN), (NKV * D, HIDDEN), (HIDDEN, NH * D)]

    def __init__(self, qw, name, n, slots, seed=0):
        import torch
        self.name, self.n, self.slots = name, n, slots
        self.shapes = self.SHAPES
        self.att = qw.Attention(NH, NKV, D, R, THETA, EPS, max_ctx=1024, max_tokens=64, max_splits=16)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + 2000)
        self.w = []
        for _ in range(slots):
            mats = []
            for rows, cols in self.shapes:
                w8 = torch.randint(-127, 128, (rows, cols), dtype=torch.int8, device="cuda", generator=g)
                sc = 0.02 * (0.5 + torch.rand((rows, cols // 32), device="cuda", generator=g))
                mats.append((w8, sc))
            self.w.append(mats)
        self.x = torch.randn((n, self.HIDDEN), device="cuda", generator=g)
        self.xo = torch.randn((n, NH * D), device="cuda", generator=g)
        self.ys = [torch.zeros((n, rows), device="cuda") for rows, _ in self.shapes]
        self.out = self.ys[0]
        self.bytes = sum(rows * cols + rows * cols // 32 * 4 for rows, cols in self.shapes)
        self.mat = True
        torch.cuda.synchronize()

    def _one(self, slot, k):
        w8, sc = self.w[slot][k]
        self.att.mat(self.xo if k == 3 else self.x, self.ys[k], w8, sc)

    def _qkv(self, slot):
        # the query + gate, key and value projections share the layer input: one qwattn_mat_multi call
        self.att.mat_multi(self.x, [(self.ys[k], *self.w[slot][k]) for k in range(3)])

    def step(self, slot):
        self._qkv(slot)
        self._one(slot, 3)

    def step_events(self, slot, ev):
        ev[0].record()
        self._qkv(slot)
        ev[1].record()
        self._one(slot, 3)
        ev[2].record()

    def main_only(self, slot):
        self._one(slot, 0)

    def close(self):
        self.w = []
        self.att.close()


class LayerWorkload(Workload):
    """A whole full-attention layer step at decode: the query + gate, key and value projections of the layer
    input (one qwattn_mat_multi call), the attention layer body (the one-launch decode), then the output
    projection, on planar Q8_0 weights of the MatWorkload shapes; every layer slot has its own cache and its
    own weights. Bytes: the K/V rows and the weights, each read once."""

    def __init__(self, qw, name, pos, n, slots, seed=0):
        import torch
        super().__init__(qw, name, pos, n, slots, 0, "f32", 0.0, seed)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + 3000)
        self.w = []
        for _ in range(slots):
            mats = []
            for rows, cols in MatWorkload.SHAPES:
                w8 = torch.randint(-127, 128, (rows, cols), dtype=torch.int8, device="cuda", generator=g)
                sc = 0.002 * (0.5 + torch.rand((rows, cols // 32), device="cuda", generator=g))
                mats.append((w8, sc))
            self.w.append(mats)
        self.x = torch.randn((n, MatWorkload.HIDDEN), device="cuda", generator=g)
        self.h = torch.zeros((n, MatWorkload.HIDDEN), device="cuda")
        self.layer = True
        self.weight_bytes = sum(rows * cols + rows * cols // 32 * 4 for rows, cols in MatWorkload.SHAPES)
        torch.cuda.synchronize()

    def _qkv(self, slot):
        n = self.n
        self.att.mat_multi(self.x, [(self.qg.view(n, -1), *self.w[slot][0]), (self.k.view(n, -1), *self.w[slot][1]),
                                    (self.v.view(n, -1), *self.w[slot][2])])

    def step(self, slot):
        self._qkv(slot)
        super().step(slot)
        self.att.mat(self.out.view(self.n, -1), self.h, *self.w[slot][3])

    def step_events(self, slot, ev):
        ev[0].record()
        self._qkv(slot)
        ev[1].record()
        super().step(slot)
        self.att.mat(self.out.view(self.n, -1), self.h, *self.w[slot][3])
        ev[2].record()


def gpu_sleep(ms):
    """Keeps the stream busy for about `ms` milliseconds, so that the launches queued behind it start
    back to back and their HIP events time the kernels, not the host's launch latency."""
    import torch
    global _SLEEP_PER_MS
    if _SLEEP_PER_MS is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_PER_MS = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(ms * _SLEEP_PER_MS))


def run_workload(wl, steps, warmup, graph):
    """Times `steps` layer steps (rotating over the slots) by wall clock, then the same kernels with
    HIP events around each one. Returns timings in microseconds."""
    import torch
    for i in range(max(warmup, wl.slots)):
        wl.step(i % wl.slots)
    torch.cuda.synchronize()
    if graph:
        # one graph holds exactly `steps` layer steps, rotating over the slots; one replay is the timed run
        wl.step(0)
        torch.cuda.synchronize()
        ref_out = wl.out.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
                for i in range(steps):
                    wl.step(i % wl.slots)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g.replay()  # untimed: the graph's first replay uploads it
        torch.cuda.synchronize()
        # a replay that computed something else than the eager step would show here
        wl.step(0)
        torch.cuda.synchronize()
        if not torch.equal(wl.out, ref_out):
            raise RuntimeError(f"{wl.name}: eager output changed after graph replays")
        timed_steps = steps
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        del g
    else:
        timed_steps = steps
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            wl.step(i % wl.slots)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0

    # per-kernel durations: HIP events on the stream the library launches on (torch's current stream),
    # queued behind a GPU sleep in batches of 16 steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for b0 in range(0, steps, 16):
        gpu_sleep(2.0)
        for i in range(b0, min(steps, b0 + 16)):
            wl.step_events(i % wl.slots, evs[i])
    torch.cuda.synchronize()
    k_first = [e[0].elapsed_time(e[1]) * 1e3 for e in evs]
    k_second = [e[1].elapsed_time(e[2]) * 1e3 for e in evs]
    k_all = [e[0].elapsed_time(e[2]) * 1e3 for e in evs]
    if not bool(torch.isfinite(wl.out).all()):
        raise RuntimeError(f"{wl.name}: non-finite attention output")
    # the dominant kernel's launch duration: batches of 16 back-to-back launches between two events on
    # the library's stream, queued behind a GPU sleep (an event between every two launches would add its
    # own cost to each figure); the mean per launch includes the in-stream gap between launches. The
    # figure is the median over KERNEL_BATCHES batches.
    per_launch = []
    for b in range(KERNEL_BATCHES):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gpu_sleep(2.0)
        e0.record()
        for i in range(16):
            wl.main_only((b * 16 + i) % wl.slots)
        e1.record()
        torch.cuda.synchronize()
        per_launch.append(e0.elapsed_time(e1) * 1e3 / 16)
    r = {"timed_steps": timed_steps, "us_per_step": wall / timed_steps * 1e6, "us_kernels": statistics.mean(k_all),
         "us_main": statistics.median(per_launch), "us_main_batches": len(per_launch),
         "us_main_min": min(per_launch)}
    if getattr(wl, "layer", False):
        r.update({"kernel": "k_mat_multi (query + gate, key, value) + k_decode_ld (attention) + k_mat_q8 (output)",
                  "us_qkv_projections": statistics.mean(k_first), "us_attention_and_output": statistics.mean(k_second),
                  "us_main_is": "k_decode_ld alone"})
    elif getattr(wl, "mat", False):
        kern = ("k_gemm<q8> (tiled MFMA GEMM, one launch a projection" if wl.n >= 16 else
                "k_mat_multi<q8> + k_mat_q8 (matrix-vector: query + gate, key and value in one launch, then output")
        r.update({"kernel": kern + "; the per-launch figure is the 8,192 x 2,048 query + gate projection alone)",
                  "us_first_event": statistics.mean(k_first)})
    elif getattr(wl, "qsa", False):
        vis, tile_keys = wl.visible()
        r.update({"kernel": "k_decode_ld<256,1,0,QSA> (one launch, visible tiles only) after k_qsa_select (raw-key append folded in: no block completes at this position)",
                  "us_indexer": statistics.mean(k_first), "us_main_each_event": statistics.mean(k_second),
                  "splits": wl.used, "visible_keys": vis, "streamed_tile_keys": tile_keys,
                  "indexer": f"{wl.IH} heads x {wl.ID} dims, blocks of {wl.CR}, budget {wl.BUDGET}"})
    elif wl.split:
        if wl.one_launch and wl.n * (NH // NKV) > 8:
            r.update({"kernel": "k_decode (fused norm+rope+append+split attend, the 16-row slices' last chunks "
                                "combining: one launch)",
                      "us_main_each_event": statistics.mean(k_first), "splits": wl.used})
        elif wl.one_launch:
            r.update({"kernel": "k_decode_ld (fused norm+rope+append+split attend, the KV heads' last chunks "
                                "combining: one launch)",
                      "us_main_each_event": statistics.mean(k_first), "splits": wl.used})
        else:
            r.update({"kernel": "k_decode (fused norm+rope+append+split attend)",
                      "us_main_each_event": statistics.mean(k_first), "us_combine": statistics.mean(k_second),
                      "splits": wl.used})
    else:
        r.update({"kernel": "k_prefill (query rows normalized and rotated in the kernel)",
                  "us_kv_norm_rope_append": statistics.mean(k_first),
                  "us_main_each_event": statistics.mean(k_second)})
    return r


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "k_decode_ld_decode_32k_k_prefill_prefill_2k_hbm_traffic.md")


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed rocprofv3 PMC summary (FETCH_SIZE +
    WRITE_SIZE, scaled by a plain copy of known size), or None when the summary does not hold it."""
    import re
    try:
        txt = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(rf"^traffic_bytes_per_launch {re.escape(kernel)} {re.escape(workload)}: (\d+)$", txt, re.M)
    return int(m.group(1)) if m else None


def cpu_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def cpu_baseline(threads, budget_s):
    """The reference CPU attention at the headline shape (32K decode, 16 Q heads) on fp32 caches, timed
    on this host: the reference's own compiled cpu_kernels.cpp primitives (oracle/_ref) when present,
    else this repository's restatement. Bounded sample: repeated calls until budget_s seconds."""
    import numpy as np
    import oracle as orc
    pos, n = 32768, 1
    r = np.random.default_rng(0)
    kc = r.standard_normal((pos + n, NKV, D), dtype=np.float32)
    vc = r.standard_normal((pos + n, NKV, D), dtype=np.float32)
    q = r.standard_normal((n, NH, D), dtype=np.float32)
    qg = r.standard_normal((n, NH, 2 * D), dtype=np.float32)
    try:
        impl, kind = orc.RefPrimitives(), "reference"
    except (FileNotFoundError, OSError):
        impl, kind = orc.Oracle(), "port"
    res = {}
    for nt in (threads, 1):
        impl.set_threads(nt)
        impl.attention(q, kc, vc, pos, qg)  # warm-up
        times = []
        t_end = time.perf_counter() + (budget_s if nt == threads else budget_s / 2)
        while time.perf_counter() < t_end and len(times) < 1000:
            t0 = time.perf_counter()
            impl.attention(q, kc, vc, pos, qg)
            times.append(time.perf_counter() - t0)
        res[nt] = (statistics.median(times), len(times))
    t, calls = res[threads]
    t1, calls1 = res[1]
    model, ncpu = cpu_info()
    byts = kv_bytes(pos + n)
    return {
        "value": round(byts / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
        "ms_per_call": round(t * 1e3, 3),
        "sample": (f"32K decode attention (n=1, 16 Q/2 KV heads, d=256, fp32 K/V cache as the reference CPU "
                   f"path), {calls} calls median, {threads} threads (16 tasks: one per Q head); "
                   f"{'reference cpu_kernels.cpp primitives compiled in place' if kind == 'reference' else 'C++ restatement'}"
                   f"; host {model}, {ncpu} CPUs visible"),
        "one_thread": {"value": round(byts / t1 / 1e9, 3), "ms_per_call": round(t1 * 1e3, 3), "calls": calls1},
        # what the reference's CPU path actually streams: every Q head reads its group's K and V rows in fp32
        "fp32_bytes_streamed": NH * 2 * (pos + n) * D * 4,
        "fp32_streamed_GBps": round(NH * 2 * (pos + n) * D * 4 / t / 1e9, 3),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--slots", type=int, default=16, help="distinct layer caches rotated at 16K/32K")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of HIP-graph replays")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--only", default="", help="comma-separated subset of workloads (for profiling)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 16 plain device copies of MIB MiB (the reference kernel for scaling PMC "
                         "FETCH_SIZE / WRITE_SIZE readings to bytes), then exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs the attention hot path on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); multi-GPU sharding is a design note, not built", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(16):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 16}))
        return
    qw = load_package()
    qw.load_library()
    graph = not args.no_graph
    only = set(filter(None, args.only.split(",")))

    configs = [
        # name, pos, n, slots, n_split (0 = one workgroup per CU), in_dtype, heavy_frac
        ("decode_32k", 32768, 1, args.slots, 0, "f32", 0.0),
        ("decode_16k", 16384, 1, args.slots, 0, "f32", 0.0),
        ("decode_16k_64splits", 16384, 1, args.slots, 64, "f32", 0.0),
        ("verify_32k_n4", 32768, 4, args.slots, 0, "f32", 0.0),
        ("decode_256k_1024splits", 262144, 1, 2, 1024, "f32", 0.01),
        ("decode_256k", 262144, 1, 2, 0, "f32", 0.01),
        ("prefill_2k_on_2k", 2048, 2048, 8, 0, "bf16", 0.0),
        # QSA layer steps (indexer + masked decode); the last field is the block size (compress ratio)
        ("decode_32k_qsa_cr4", 32768, 1, args.slots, 0, "f32", 4),
        ("decode_32k_qsa_cr64", 32768, 1, args.slots, 0, "f32", 64),
        ("decode_256k_qsa_cr4", 262144, 1, 2, 0, "f32", 4),
        ("decode_256k_qsa_cr64", 262144, 1, 2, 0, "f32", 64),
        # the layer's projections (planar Q8_0 weights), one decode token and a 4-token verify pass
        ("proj_q8_n1", 0, 1, args.slots, 0, "f32", 0.0),
        ("proj_q8_n4", 0, 4, args.slots, 0, "f32", 0.0),
        # and a 2,048-token prefill chunk (the tiled MFMA GEMM)
        ("proj_q8_n2048", 0, 2048, 8, 0, "f32", 0.0),
        # the whole full-attention layer at decode: projections around the attention body
        ("layer_32k_q8", 32768, 1, args.slots, 0, "f32", 0.0),
    ]
    results = {}
    for name, pos, n, slots, n_split, dt, heavy in configs:
        if only and name not in only:
            continue
        print(f"[bench] {name}: pos={pos} n={n} slots={slots} splits={n_split or 'auto'}", file=sys.stderr,
              flush=True)
        if name.startswith("proj_"):
            wl = MatWorkload(qw, name, n, slots, seed=len(results))
        elif name.startswith("layer_"):
            wl = LayerWorkload(qw, name, pos, n, slots, seed=len(results))
        elif "_qsa" in name:
            wl = QsaWorkload(qw, name, pos, n, slots, int(heavy), seed=len(results))
        else:
            wl = Workload(qw, name, pos, n, slots, n_split, dt, heavy, seed=len(results))
        r = run_workload(wl, args.steps, args.warmup, graph)
        wl_bytes = getattr(wl, "bytes", 0)
        wl_weight_bytes = getattr(wl, "weight_bytes", 0)
        wl.close()
        del wl
        torch.cuda.empty_cache()
        if name.startswith("proj_") and n >= 16:
            # 2 n rows cols flops a projection; the per-launch figure is the 8,192 x 2,048 projection's
            flops = 2 * n * sum(rows * cols for rows, cols in MatWorkload.SHAPES)
            r["value"] = flops / (r["us_per_step"] * 1e-6) / 1e12
            r["unit"] = "TFLOP/s"
            r["algorithmic_flops"] = flops
            r["frac_mfma_step"] = flops / (r["us_per_step"] * 1e-6) / MFMA_F16_PEAK
            r["frac_mfma_kernel"] = 2 * n * NH * 2 * D * 2048 / (r["us_main"] * 1e-6) / MFMA_F16_PEAK
        elif name.startswith("layer_"):
            # the K/V rows and the weights, each read once a step; us_first_event = the q/k/v projections
            byts = kv_bytes(pos + n) + wl_weight_bytes
            r["value"] = byts / (r["us_per_step"] * 1e-6) / 1e9
            r["unit"] = "GB/s (K/V + weights)"
            r["algorithmic_bytes"] = byts
            r["frac_hbm_step"] = byts / (r["us_per_step"] * 1e-6) / HBM_PEAK
        elif name.startswith("proj_"):
            # the weights read once; the per-launch figure is the largest projection's
            r["value"] = wl_bytes / (r["us_per_step"] * 1e-6) / 1e9
            r["unit"] = "GB/s (weights)"
            r["algorithmic_bytes"] = wl_bytes
            r["frac_hbm_step"] = wl_bytes / (r["us_per_step"] * 1e-6) / HBM_PEAK
            q_bytes = NH * 2 * D * 2048 * (1 + 4 / 32)
            r["frac_hbm_kernel"] = q_bytes / (r["us_main"] * 1e-6) / HBM_PEAK
        elif "_qsa" in name:
            # the K/V bytes of the keys the selection leaves visible (each fp16 row once)
            byts = 2 * r["visible_keys"] * NKV * D * 2
            r["value"] = byts / (r["us_per_step"] * 1e-6) / 1e9
            r["unit"] = "GB/s (visible keys)"
            r["algorithmic_bytes"] = byts
            r["frac_hbm_kernel"] = byts / (r["us_main"] * 1e-6) / HBM_PEAK
            dense = results.get("decode_256k" if pos == 262144 else "decode_32k")  # the dense step at this length
            if dense:
                r["step_speedup_vs_dense"] = dense["us_per_step"] / r["us_per_step"]
        elif n * (NH // NKV) <= 32:
            byts = kv_bytes(pos + n)
            r["value"] = byts / (r["us_per_step"] * 1e-6) / 1e9
            r["unit"] = "GB/s"
            r["frac_hbm_step"] = byts / (r["us_per_step"] * 1e-6) / HBM_PEAK
            r["frac_hbm_kernel"] = byts / (r["us_main"] * 1e-6) / HBM_PEAK
            r["algorithmic_bytes"] = byts
        else:
            fl = causal_flops(pos, n)
            r["value"] = fl / (r["us_per_step"] * 1e-6) / 1e12
            r["unit"] = "TFLOP/s"
            r["frac_mfma_step"] = fl / (r["us_per_step"] * 1e-6) / MFMA_F16_PEAK
            r["frac_mfma_kernel"] = fl / (r["us_main"] * 1e-6) / MFMA_F16_PEAK
            r["algorithmic_flops"] = fl
        if n * (NH // NKV) <= 32 and "_qsa" not in name and not name.startswith("proj_"):
            r["splits_requested"] = n_split or "auto"
        results[name] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        print(f"[bench] {name}: {json.dumps(results[name])}", file=sys.stderr, flush=True)

    head = results.get("decode_32k")
    cpu = None
    if not args.no_cpu and (not only or "decode_32k" in only):
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(threads=min(16, os.cpu_count() or 1), budget_s=args.cpu_seconds)
    line = {
        "metric": "decode attn KV GB/s (% HBM peak) @32K ctx; prefill TFLOP/s (% MFMA peak)",
        "value": round(head["value"], 3) if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["timed_steps"] if head else args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 6) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 KV / fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V caches and projections)",
        "config": {"workload": "decode_32k: Qwen3-Next full-attention layer body (norm+rope+append, split-KV "
                               "attend, LSE combine), batch 1, 32,768 cached tokens + 1",
                   "heads": "16q/2kv", "head_dim": D, "rope_dim": R, "kv_cache": "fp16",
                   "layer_caches_rotated": args.slots, "timing": "hip-graph replay" if graph else "eager"},
        "roofline": None,
        "cpu_baseline": cpu,
        "workloads": results,
    }
    if head:
        # dim slices per combined row, as the library picks them (combine_slices in csrc/qwattn.cpp)
        nds = next((k for k in (4, 2) if 2 * (NH // NKV) * k <= head["splits"]), 1)
        line["roofline"] = {"bound": "hbm",
                            "kernel": f"k_decode_ld<256,1,0> (one launch: {head['splits']}x{NKV} streaming "
                                      f"workgroups, the last {NH // NKV * nds} of each KV head combining a "
                                      f"{256 // nds}-dim slice of one output row each)",
                            "achieved": round(head["algorithmic_bytes"] / (head["us_main"] * 1e-6) / 1e9, 2),
                            "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                            "frac": round(head["frac_hbm_kernel"], 4),
                            "traffic": measured_traffic("k_decode_ld", "decode_32k"),
                            "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
                            "kernel_us": head["us_main"]}
    pf = results.get("prefill_2k_on_2k")
    if pf:
        line["prefill_roofline"] = {"bound": "mfma",
                                    "kernel": "k_prefill<256,1,true> (query rows normalized and rotated in the "
                                              "kernel from bf16 projections, bf16 gate; 8 waves x 16 rows, two a SIMD, 16x16x32 "
                                              "MFMAs; paired schedule, grid 256)",
                                    "achieved": round(pf["algorithmic_flops"] / (pf["us_main"] * 1e-6) / 1e12, 2),
                                    "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                                    "frac": round(pf["frac_mfma_kernel"], 4),
                                    "traffic": measured_traffic("k_prefill", "prefill_2k_on_2k"),
                                    "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
                                    "kernel_us": pf["us_main"]}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
