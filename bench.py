#!/usr/bin/env python3
"""Benchmark of the quantized matrix-vector path on one MI355X.

Default workload: the Q4_0 FFN of one decode token (gate/up W 8192x2048, down W
2048x8192, x ~ N(0,1)).  A step is h = gelu(W_gate x) * (W_up x) followed by
y = W_down h -- two launches of libg4hip.so.  Weights are resident in HBM before
timing starts; each step uses the next of several weight copies whose total
exceeds twice the 256 MB Infinity Cache, so every step streams from HBM.
The timed steps are captured in one HIP graph (a replay's own launch cost is
spread over the steps, as in a decode loop) and replayed once; the timed region
is bracketed by device synchronisation.

Prints one JSON line.  `value` is GB/s of algorithmic bytes (each weight and
activation byte counted once) per second; `roofline` covers the dominant
kernel, timed with HIP events on the launch stream; `cpu_baseline` times the
oracle's restatement of the reference's 512-bit Vector API path on the host
cores over a bounded sample of the same workload.

Other workloads: --workload q8_0_matvec | q4_0_ffn | q8_0_lm_head |
q4_k_batched[:M] | moe[:T] | q5_k_matvec | q6_k_matvec | q4_0_ffn_block (the
FFN with its norms and residual add) | q8_0_lm_head_cap (final norm, soft-cap,
arg-max) | attention[:L] (decode attention over L cached positions); --all prints
one line per workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gemma4.kt_amd"))

import numpy as np  # noqa: E402

METRIC = "quant matvec GB/s & % of HBM peak (Q8_0/Q4_0/Q4_K); MoE expert tokens/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 matrix-core peak
MALL_BYTES = 256 << 20
Q8_0, Q4_0, Q4_K = 8, 2, 12


# HBM bytes per launch of each workload's timed kernel (or launch group), from two
# rocprofv3 --pmc passes over `bench.py --eager`: FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0
# (KiB), the factors being what the counters read for a plain 256 MiB fp32 copy.
# Recorded in profiles/hbm_traffic_fetch_write_size.md (same command and kernels).
# "name:part" keys give the other separately timed launches of a step.
TRAFFIC_BYTES = {
    "q4_0_ffn_decode_token": 19186432,
    "q4_0_ffn_decode_token:down": 9835392,
    "q8_0_matvec_2048x2048": 4638592,
    "q8_0_lm_head_262144x2048_argmax": 572062368,
    "q4_k_batched_8192x2048_m1": 9671552,
    "q4_k_batched_8192x2048_m8": 10462208,
    "q4_k_batched_8192x2048_m32": 12698240,
    "q4_k_batched_8192x2048_m64": 15843968,
    "moe_q4_k_128x(2816x2048+2048x1408)_top8_t1": 40018112,
    "moe_q4_k_128x(2816x2048+2048x1408)_top8_t16": 479384304,
    "moe_q4_k_128x(2816x2048+2048x1408)_top8_t128": 727389920,
    "q5_k_matvec_8192x2048": 11777024,
    "q6_k_matvec_8192x2048": 14138240,
    "q4_0_ffn_block_decode_token": 29151872,
    "q8_0_lm_head_262144x2048_norm_softcap_argmax": 572338944,
    "attention_decode_h16_kv8_d256_len8192": 136771584,
}


def copies_for(nbytes: int, cap: int = 256) -> int:
    """Weight copies so that one pass over them spans >= 2x the Infinity Cache."""
    if nbytes >= 2 * MALL_BYTES:
        return 1
    return max(2, min(cap, math.ceil(2 * MALL_BYTES / nbytes)))


class Workload:
    """Device buffers + the per-step launch sequence of one workload."""

    name = ""
    unit = "GB/s"
    step_bytes = 0          # algorithmic bytes per step
    dominant_name = ""           # dominant kernel name (as rocprof reports it)
    dominant_bytes = 0      # algorithmic bytes per launch of the dominant kernel
    bound = "hbm"           # roofline the dominant kernel is judged against ("hbm" or "mfma")
    dominant_flops = 0      # useful flops per launch (bound "mfma")
    tokens_per_step = 0     # MoE: tokens per step
    copies = 1
    # True: the dominant launch group is the whole step, so its time per launch is
    # the timed region's own, from HIP events around it (no separate timing)
    dominant_is_step = True

    def step(self, i: int) -> None:
        """Launch one step on weight copy / routing i (device work only, graph-capturable)."""
        raise NotImplementedError

    def dominant(self, i: int) -> None:
        """Launch only the dominant kernel of step i (for its roofline timing)."""
        self.step(i)

    def set_steps(self, steps: int) -> None:
        """The timed region runs steps 0 .. steps-1 (workloads whose bytes differ per step adjust)."""

    def parts(self) -> list:
        """(kernel name, algorithmic bytes per launch, launch fn(i), traffic key) of each
        launch of a step that is timed on its own; by default the dominant kernel only."""
        return [(self.dominant_name, self.dominant_bytes, self.dominant, self.name)]

    # The same step through the host-pointer entry point (activations copied in,
    # results copied out, synchronous), timed apart from `value`; None: no such call.
    host_step = None

    def cpu_step(self) -> None:
        raise NotImplementedError

    def config(self) -> dict:
        raise NotImplementedError


class FfnQ4_0(Workload):
    name = "q4_0_ffn_decode_token"
    dominant_name = "k_rows<FmtQ4_0, 32, EPI_GELU_PAIR> (gate+up fused)"
    down_name = "k_wide<FmtQ4_0, 32, 4, 2> (down)"
    dominant_is_step = False  # gate+up and down timed apart

    def __init__(self, g4, ctx, torch):
        import synth
        c = synth.q4_0_ffn()
        self.c = c
        dim, hidden = c["dim"], c["hidden"]
        self.dim, self.hidden = dim, hidden
        wbytes = c["gate"].nbytes + c["up"].nbytes + c["down"].nbytes
        self.copies = copies_for(wbytes)
        self.w = []
        for _ in range(self.copies):
            self.w.append(tuple(g4.FloatTensorFactory.create(ctx, Q4_0, c[k], n)
                                for k, n in (("gate", hidden * dim), ("up", hidden * dim), ("down", dim * hidden))))
        self.x = torch.from_numpy(c["x"]).cuda()
        self.h = torch.empty(hidden, dtype=torch.float32, device="cuda")
        self.y = torch.empty(dim, dtype=torch.float32, device="cuda")
        # algorithmic bytes as quoted for this workload: the 3 weight matrices plus
        # 122880 B of activations (x read by gate and up, gate/up written, h read, y written)
        self.step_bytes = wbytes + 4 * (2 * dim + 2 * hidden + hidden + dim)
        # fused gate+up launch: both matrices, x once, h written once
        self.dominant_bytes = c["gate"].nbytes + c["up"].nbytes + 4 * dim + 4 * hidden
        self.g4, self.ctx = g4, ctx

    def step(self, i):
        wg, wu, wd = self.w[i % self.copies]
        self.g4.ffn_gate_up_dev(self.ctx, wg, wu, self.x, self.h, self.dim, self.hidden)
        wd.matmul_dev(self.h, self.y, self.dim, self.hidden)

    def host_step(self, i):
        wg, wu, wd = self.w[i % self.copies]
        self.g4.ffn(self.ctx, wg, wu, wd, self.c["x"], self.dim, self.hidden)

    def dominant(self, i):
        wg, wu, _ = self.w[i % self.copies]
        self.g4.ffn_gate_up_dev(self.ctx, wg, wu, self.x, self.h, self.dim, self.hidden)

    def down(self, i):
        self.w[i % self.copies][2].matmul_dev(self.h, self.y, self.dim, self.hidden)

    def parts(self):
        # the down launch: W_down, h read once, y written once
        down_bytes = self.c["down"].nbytes + 4 * self.hidden + 4 * self.dim
        return [(self.dominant_name, self.dominant_bytes, self.dominant, self.name),
                (self.down_name, down_bytes, self.down, self.name + ":down")]

    def cpu_setup(self, oracle):
        self.oracle = oracle
        self.gu_cat = np.concatenate([self.c["gate"], self.c["up"]])
        self.ids = np.zeros((1, 1), np.int32)
        self.one = np.ones((1, 1), np.float32)

    def cpu_step(self):
        self.oracle.moe(Q4_0, self.gu_cat, Q4_0, self.c["down"], self.c["x"].reshape(1, -1), self.ids, self.one,
                        self.dim, self.hidden)

    def config(self):
        return {"workload": self.name, "format": "Q4_0", "gate_up": [self.hidden, self.dim],
                "down": [self.dim, self.hidden], "algorithmic_bytes_per_step": self.step_bytes,
                "weight_copies": self.copies}


class MatvecQ8_0(Workload):
    name = "q8_0_matvec_2048x2048"
    dominant_name = "k_rows<FmtQ8_0, 32, EPI_STORE>"

    def __init__(self, g4, ctx, torch):
        import synth
        c = synth.q8_0_matvec_2048()
        self.c = c
        self.copies = copies_for(c["w"].nbytes)
        self.w = [g4.FloatTensorFactory.create(ctx, Q8_0, c["w"], 2048 * 2048) for _ in range(self.copies)]
        self.x = torch.from_numpy(c["x"]).cuda()
        self.y = torch.empty(2048, dtype=torch.float32, device="cuda")
        self.yh = np.empty(2048, np.float32)
        self.step_bytes = c["w"].nbytes + 4 * 2048 * 2
        self.dominant_bytes = self.step_bytes

    def step(self, i):
        self.w[i % self.copies].matmul_dev(self.x, self.y, 2048, 2048)

    def host_step(self, i):
        self.w[i % self.copies].matmul(self.c["x"], self.yh, 2048, 2048)

    def cpu_setup(self, oracle):
        self.oracle = oracle

    def cpu_step(self):
        self.oracle.matmul(Q8_0, self.c["w"], self.c["x"], 2048, 2048)

    def config(self):
        return {"workload": self.name, "format": "Q8_0", "w": [2048, 2048],
                "algorithmic_bytes_per_step": self.step_bytes, "weight_copies": self.copies}


class LmHeadQ8_0(Workload):
    name = "q8_0_lm_head_262144x2048_argmax"
    dominant_name = "k_rows<FmtQ8_0, 32, EPI_ARGMAX> + k_argmax_final"

    def __init__(self, g4, ctx, torch):
        import synth
        c = synth.q8_0_lm_head()
        self.c = c
        V, D = c["dim0"], c["dim1"]
        self.V, self.D = V, D
        self.copies = copies_for(c["w"].nbytes)
        self.w = [g4.FloatTensorFactory.create(ctx, Q8_0, c["w"], V * D) for _ in range(self.copies)]
        self.x = torch.from_numpy(c["x"]).cuda()
        self.logits = torch.empty(V, dtype=torch.float32, device="cuda")
        self.idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.lh = np.empty(V, np.float32)
        self.step_bytes = c["w"].nbytes + 4 * D + 4 * V + 4
        self.dominant_bytes = self.step_bytes

    def step(self, i):
        self.w[i % self.copies].matmul_argmax_dev(self.x, self.logits, self.idx.data_ptr(), self.V, self.D)

    def host_step(self, i):
        self.w[i % self.copies].matmul_argmax(self.c["x"], self.V, self.D, logits=self.lh)

    def cpu_setup(self, oracle):
        self.oracle = oracle

    def cpu_step(self):
        lg = self.oracle.matmul(Q8_0, self.c["w"], self.c["x"], self.V, self.D)
        self.oracle.argmax(lg)

    def cpu_sample_rows(self):
        return 16384  # bounded CPU sample: a slice of the vocabulary rows

    def cpu_step_rows(self, rows):
        lg = self.oracle.matmul(Q8_0, self.c["w"], self.c["x"], rows, self.D)
        self.oracle.argmax(lg)

    def config(self):
        return {"workload": self.name, "format": "Q8_0", "w": [self.V, self.D],
                "algorithmic_bytes_per_step": self.step_bytes, "weight_copies": self.copies}


class BatchedQ4_K(Workload):
    def __init__(self, g4, ctx, torch, m=8):
        import synth
        c = synth.q4_k_batched(m)
        self.c, self.m = c, m
        # one or two tokens: the row-stream kernel (one segment per token); three or
        # more: the matrix-core kernel (one column split up to 2048 columns, more
        # splits summed by k_tok_reduce), its HALF form (token rows 8..15 not
        # loaded) up to eight tokens; the 16 q operands (SUB8) up to eight tokens and
        # from four row tiles per workgroup; whole slices and row tiles (FULL) here
        self.dominant_name = ("k_rows<FmtQ4_K, 32, EPI_STORE, KSEL>" if m <= 2 else
                              "k_tok_q4k<1, 16, true, %s, true> (bf16x3 MFMA 16x16x32)" % (
                                  "true, true" if m <= 8 else "false, true" if m > 16 else "false, false"))
        self.name = "q4_k_batched_8192x2048_m%d" % m
        R, D = c["dim0"], c["dim1"]
        self.R, self.D = R, D
        self.copies = copies_for(c["w"].nbytes)
        self.w = [g4.FloatTensorFactory.create(ctx, Q4_K, c["w"], R * D) for _ in range(self.copies)]
        self.X = torch.from_numpy(np.ascontiguousarray(c["x"])).cuda()
        self.Y = torch.empty((m, R), dtype=torch.float32, device="cuda")
        self.step_bytes = c["w"].nbytes + 4 * m * (D + R)
        self.dominant_bytes = self.step_bytes
        self.dominant_flops = 2 * m * R * D
        # arithmetic intensity 3.6 M flop/B: past the HBM ridge of the exact-fp32
        # scheme (three bf16 products per weight) from M = 32 on
        self.bound = "mfma" if m >= 32 else "hbm"

    def step(self, i):
        self.w[i % self.copies].matmul_batch_dev(self.X, self.m, self.Y, self.R, self.D)

    def host_step(self, i):
        self.w[i % self.copies].matmul_batch(np.ascontiguousarray(self.c["x"]), self.R, self.D)

    def cpu_setup(self, oracle):
        self.oracle = oracle

    def cpu_step(self):
        for i in range(self.m):
            self.oracle.matmul(Q4_K, self.c["w"], self.c["x"][i], self.R, self.D)

    def config(self):
        return {"workload": self.name, "format": "Q4_K", "w": [self.R, self.D], "m": self.m,
                "algorithmic_bytes_per_step": self.step_bytes, "weight_copies": self.copies,
                "flops_per_step": 2 * self.m * self.R * self.D}


class MoeQ4_K(Workload):
    unit = "tokens/s"

    def __init__(self, g4, ctx, torch, tokens=1, routings=32):
        import synth
        self.T = tokens
        self.name = "moe_q4_k_128x(2816x2048+2048x1408)_top8_t%d" % tokens
        # up to 40 tokens: the down projection and the weighted sum share a launch
        # (one row step per wave for one token, looped row steps for more); 41 or
        # more tokens: a routing launch, then the experts grouped on the matrix cores
        # (16-pair tiles: gate and up rows, gelu, down), then the weighted sum
        if tokens >= 41:
            self.dominant_name = ("g4_moe_routed: k_route + k_grp_q4k<true> (gate+up rows) + k_gelu_mul4 + "
                                  "k_grp_q4k<true> (down) (experts grouped on the matrix cores) + k_moe_combine")
        else:
            self.dominant_name = (("g4_moe_routed: k_rows<FmtQ4_K, 32, EPI_GELU_PAIR, ROUTE, KSEL> (routing + gate_up) + "
                                   "k_moe_down_xl<FmtQ4_K> (down + weighted sum)") if tokens == 1 else
                                  ("g4_moe_routed: k_rows<FmtQ4_K, 32, EPI_GELU_PAIR, ROUTE, 8 waves, SLOTW, KSEL> "
                                   "(routing + gate_up) + k_moe_down_xlt<FmtQ4_K, STEP> (down + weighted sum)"))
        base = synth.moe_q4_k(tokens)
        E, D, FF, K = base["n_experts"], base["dim"], base["ff"], base["k"]
        self.E, self.D, self.FF, self.K = E, D, FF, K
        self.base = base
        per_expert = (2 * FF * D + D * FF) // 256 * 144
        self.copies = routings
        self.logits, self.X, self.distinct, self.lgh, self.Xh = [], [], [], [], []
        for r in range(routings):  # routing r = the logits/x streams of synth.moe_q4_k(tokens, routing_seed=r)
            lg = synth.activations(synth.SEED_MOE_Q4_K, "router%d.%d" % (tokens, r), tokens * E).reshape(tokens, E)
            x = synth.activations(synth.SEED_MOE_Q4_K, "x%d.%d" % (tokens, r), tokens * D).reshape(tokens, D)
            ids, _ = g4.moe_route(ctx, lg, K, True)
            self.distinct.append(len(np.unique(ids)))
            self.logits.append(torch.from_numpy(lg).cuda())
            self.X.append(torch.from_numpy(x).cuda())
            self.lgh.append(lg)
            self.Xh.append(x)
        self.ids = torch.zeros((tokens, K), dtype=torch.int32, device="cuda")
        self.gw = torch.zeros((tokens, K), dtype=torch.float32, device="cuda")
        self.Y = torch.empty((tokens, D), dtype=torch.float32, device="cuda")
        self.per_expert = per_expert
        mean_distinct = float(np.mean(self.distinct))
        # expert slab copies: step i reads copy i mod n, with n such that the n - 1
        # steps between two uses of one copy stream more than twice the Infinity
        # Cache (all of a step's experts, from HBM, every step)
        step_experts = mean_distinct * per_expert
        self.n_slabs = (1 if step_experts >= 2 * MALL_BYTES else
                        int(math.ceil(2 * MALL_BYTES / step_experts)) + 1)
        self.slabs = [(g4.FloatTensorFactory.create(ctx, Q4_K, base["gate_up"], E * 2 * FF * D),
                       g4.FloatTensorFactory.create(ctx, Q4_K, base["down"], E * D * FF))
                      for _ in range(self.n_slabs)]
        # a step reads every routed expert's gate_up and down once, x and the router
        # logits, and writes Y (the routing outputs are 8 bytes per slot)
        self.step_bytes = int(mean_distinct * per_expert + 4 * tokens * (D + E + D))
        self.dominant_bytes = self.step_bytes
        self.tokens_per_step = tokens
        self.g4, self.ctx = g4, ctx

    def set_steps(self, steps):
        # the routings the timed steps use (step i takes routing i mod copies)
        used = [self.distinct[i % self.copies] for i in range(steps)]
        self.mean_used = float(np.mean(used))
        self.step_bytes = int(self.mean_used * self.per_expert + 4 * self.T * (self.D + self.E + self.D))
        self.dominant_bytes = self.step_bytes

    def step(self, i):
        # routing (inside the gate_up launch), experts and the weighted sum
        r = i % self.copies
        wgu, wdn = self.slabs[i % self.n_slabs]
        self.g4.moe_routed_dev(self.ctx, wgu, wdn, self.X[r], self.T, self.D, self.FF, self.logits[r],
                               self.E, self.K, True, self.ids.data_ptr(), self.gw, self.Y)

    def host_step(self, i):
        r = i % self.copies
        wgu, wdn = self.slabs[i % self.n_slabs]
        self.g4.moe_routed(self.ctx, wgu, wdn, self.Xh[r], self.lgh[r], self.K, True, self.D, self.FF)

    def cpu_setup(self, oracle):
        self.oracle = oracle
        self.cpu_ids, self.cpu_w = oracle.route(self.base["logits"], self.K, True)

    def cpu_step(self):
        self.oracle.moe(Q4_K, self.base["gate_up"], Q4_K, self.base["down"], self.base["x"], self.cpu_ids,
                        self.cpu_w, self.D, self.FF)

    def config(self):
        return {"workload": self.name, "format": "Q4_K", "experts": self.E, "top_k": self.K, "tokens": self.T,
                "routings": self.copies, "slab_copies": self.n_slabs,
                "mean_distinct_experts": getattr(self, "mean_used", float(np.mean(self.distinct))),
                "algorithmic_bytes_per_step": self.step_bytes}


class MatvecKQuant(Workload):
    """Single-token matvec of an 8192x2048 Q5_K or Q6_K matrix (the K-quants a
    llama.cpp mix pairs with Q4_K; no reference configuration, measured for parity
    of coverage): x ~ N(0,1), y = W x."""

    def __init__(self, g4, ctx, torch, ggml_type):
        import synth
        self.t = ggml_type
        fmt = {13: "q5_k", 14: "q6_k"}[ggml_type]
        self.name = "%s_matvec_8192x2048" % fmt
        self.dominant_name = "k_rows<Fmt%s, 32, EPI_STORE>" % fmt.upper()
        self.R, self.D = 8192, 2048
        self.raw = synth.weights(0x51A5, fmt, ggml_type, self.R * self.D)
        self.xh = synth.activations(0x51A5, "x", self.D)
        self.copies = copies_for(self.raw.nbytes)
        self.w = [g4.FloatTensorFactory.create(ctx, ggml_type, self.raw, self.R * self.D) for _ in range(self.copies)]
        self.x = torch.from_numpy(self.xh).cuda()
        self.y = torch.empty(self.R, dtype=torch.float32, device="cuda")
        self.yh = np.empty(self.R, np.float32)
        self.step_bytes = self.dominant_bytes = self.raw.nbytes + 4 * (self.D + self.R)
        self.fmt = fmt

    def step(self, i):
        self.w[i % self.copies].matmul_dev(self.x, self.y, self.R, self.D)

    def host_step(self, i):
        self.w[i % self.copies].matmul(self.xh, self.yh, self.R, self.D)

    def cpu_setup(self, oracle):
        self.oracle = oracle

    def cpu_step(self):
        self.oracle.matmul(self.t, self.raw, self.xh, self.R, self.D)

    def config(self):
        return {"workload": self.name, "format": self.fmt.upper(), "w": [self.R, self.D],
                "algorithmic_bytes_per_step": self.step_bytes, "weight_copies": self.copies}


class FfnBlockQ4_0(Workload):
    """The Q4_0 FFN as a whole dense decode block (Llama.kt:355-363): pre-norm
    fused into the gate/up launch, down, then post-norm plus residual add, with
    the residual stream x updated in place in device memory."""
    name = "q4_0_ffn_block_decode_token"
    dominant_name = ("launch group of g4_ffn_block: k_rows<FmtQ4_0, 32, EPI_GELU_PAIR, NORM> + "
                     "k_wide<FmtQ4_0, 32, 4, 2> + k_rmsnorm_v (residual)")

    def __init__(self, g4, ctx, torch):
        import synth
        c = synth.q4_0_ffn_block()
        self.c = c
        dim, hidden = c["dim"], c["hidden"]
        self.dim, self.hidden, self.eps = dim, hidden, c["eps"]
        wbytes = c["gate"].nbytes + c["up"].nbytes + c["down"].nbytes
        self.copies = copies_for(wbytes)
        F = g4.FloatTensorFactory.create
        self.w = []
        for _ in range(self.copies):
            self.w.append(tuple(F(ctx, Q4_0, c[k], n) for k, n in
                                (("gate", hidden * dim), ("up", hidden * dim), ("down", dim * hidden))))
        self.n_pre = F(ctx, 0, c["norm_pre"], dim)
        self.n_post = F(ctx, 0, c["norm_post"], dim)
        self.x = torch.from_numpy(c["x"]).cuda()
        # weights plus activations: gate/up launch reads x and the pre-norm weight and
        # writes h; down reads h and writes y; the residual launch reads y, the
        # post-norm weight and x and writes y and x
        self.step_bytes = wbytes + 4 * (8 * dim + 2 * hidden)
        self.dominant_bytes = self.step_bytes
        self.g4, self.ctx = g4, ctx

    def step(self, i):
        wg, wu, wd = self.w[i % self.copies]
        self.g4.ffn_block_dev(self.ctx, wg, wu, wd, self.n_pre, self.n_post, self.x, self.dim, self.hidden,
                              self.eps)

    def host_step(self, i):
        wg, wu, wd = self.w[i % self.copies]
        self.g4.ffn_block(self.ctx, wg, wu, wd, self.n_pre, self.n_post, self.c["x"], self.dim, self.hidden,
                          self.eps)

    def cpu_setup(self, oracle):
        self.oracle = oracle

    def cpu_step(self):
        c = self.c
        self.oracle.ffn_block(Q4_0, c["gate"], Q4_0, c["up"], Q4_0, c["down"], c["norm_pre"], c["norm_post"],
                              c["x"], self.dim, self.hidden, self.eps)

    def config(self):
        return {"workload": self.name, "format": "Q4_0", "gate_up": [self.hidden, self.dim],
                "down": [self.dim, self.hidden], "norms": "F32 pre/post", "eps": self.eps,
                "algorithmic_bytes_per_step": self.step_bytes, "weight_copies": self.copies}


class LmHeadCapQ8_0(LmHeadQ8_0):
    """The Q8_0 LM head behind its final norm and logit soft-cap (Llama.kt:401-407)
    plus the greedy pick: norm fused into the matvec, cap and arg-max in its epilogue."""
    name = "q8_0_lm_head_262144x2048_norm_softcap_argmax"
    dominant_name = "k_rows<FmtQ8_0, 32, EPI_ARGMAX, NORM> (softcap) + k_argmax_final"

    def __init__(self, g4, ctx, torch):
        import synth
        c = synth.q8_0_lm_head_block()
        self.c = c
        V, D = c["dim0"], c["dim1"]
        self.V, self.D, self.eps, self.cap = V, D, c["eps"], c["cap"]
        self.copies = copies_for(c["w"].nbytes)
        self.w = [g4.FloatTensorFactory.create(ctx, Q8_0, c["w"], V * D) for _ in range(self.copies)]
        self.norm = g4.FloatTensorFactory.create(ctx, 0, c["norm"], D)
        self.x = torch.from_numpy(c["x"]).cuda()
        self.logits = torch.empty(V, dtype=torch.float32, device="cuda")
        self.idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.step_bytes = c["w"].nbytes + 4 * D + 4 * D + 4 * V + 4
        self.dominant_bytes = self.step_bytes
        self.g4, self.ctx = g4, ctx

    def step(self, i):
        self.g4.lm_head_dev(self.ctx, self.w[i % self.copies], self.norm, self.x, self.logits,
                            self.idx.data_ptr(), self.V, self.D, self.eps, self.cap)

    def host_step(self, i):
        self.g4.lm_head(self.ctx, self.w[i % self.copies], self.norm, self.c["x"], self.V, self.D, self.eps,
                        self.cap)

    def cpu_step(self):
        self.cpu_step_rows(self.V)

    def cpu_step_rows(self, rows):
        c = self.c
        self.oracle.lm_head(Q8_0, c["w"], c["norm"], c["x"], rows, self.D, self.eps, self.cap)

    def config(self):
        return {"workload": self.name, "format": "Q8_0", "w": [self.V, self.D], "norm": "F32", "eps": self.eps,
                "softcap": self.cap, "algorithmic_bytes_per_step": self.step_bytes, "weight_copies": self.copies}


class AttentionDecode(Workload):
    """Decode attention of one token over one layer's KV cache (Llama.kt:198-218):
    16 query heads sharing 8 kv heads of size 256, fp32 caches of `length` rows."""
    dominant_name = "k_att_part<256, 2> + k_att_combine"

    def __init__(self, g4, ctx, torch, length: int):
        import synth
        self.H, self.KV, self.HS, self.Lc = 16, 8, 256, length
        kv_dim = self.KV * self.HS
        self.name = "attention_decode_h16_kv8_d256_len%d" % length
        self.q_np = synth.activations(0xA77, "q", self.H * self.HS)
        self.k_np = synth.activations(0xA77, "k", length * kv_dim)
        self.v_np = synth.activations(0xA77, "v", length * kv_dim)
        cache_bytes = 2 * self.k_np.nbytes
        self.copies = copies_for(cache_bytes, cap=64)
        self.q = torch.from_numpy(self.q_np).cuda()
        self.kc = [torch.from_numpy(self.k_np).cuda() for _ in range(self.copies)]
        self.vc = [torch.from_numpy(self.v_np).cuda() for _ in range(self.copies)]
        self.out = torch.empty(self.H * self.HS, dtype=torch.float32, device="cuda")
        # K and V rows once each, q read, out written
        self.step_bytes = cache_bytes + 2 * 4 * self.H * self.HS
        self.dominant_bytes = self.step_bytes
        self.g4, self.ctx = g4, ctx

    def step(self, i):
        c = i % self.copies
        self.g4.attention_dev(self.ctx, self.q, self.kc[c], self.vc[c], self.out, self.H, self.KV, self.HS,
                              self.Lc - 1, 0)

    def cpu_setup(self, oracle):
        self.oracle = oracle

    def cpu_step(self):
        self.oracle.attention(self.q_np, self.k_np, self.v_np, self.H, self.KV, self.HS, self.Lc - 1, 0)

    def config(self):
        return {"workload": self.name, "n_heads": self.H, "n_kv_heads": self.KV, "head_size": self.HS,
                "positions": self.Lc, "cache": "fp32", "algorithmic_bytes_per_step": self.step_bytes,
                "cache_copies": self.copies}


class CopyCalibration(Workload):
    """A plain fp32 copy of known size (y = x * 1 through torch's elementwise kernel).

    Not part of --all: it is the reference point that scales the FETCH_SIZE /
    WRITE_SIZE counters into HBM bytes (each counter divided by what it reads
    for exactly 256 MiB in and 256 MiB out)."""
    name = "copy_256MiB_f32"
    dominant_name = "vectorized_elementwise_kernel (y = x * 1)"

    def __init__(self, g4, ctx, torch):
        n = 64 << 20
        self.x = torch.ones(n, dtype=torch.float32, device="cuda")
        self.y = torch.empty_like(self.x)
        self.step_bytes = self.dominant_bytes = 2 * 4 * n
        self.torch = torch

    def step(self, i):
        self.torch.mul(self.x, 1.0, out=self.y)

    def config(self):
        return {"workload": self.name, "bytes_read": self.step_bytes // 2, "bytes_written": self.step_bytes // 2}


def make_workload(spec: str, g4, ctx, torch) -> Workload:
    name, _, arg = spec.partition(":")
    if name == "copy":
        return CopyCalibration(g4, ctx, torch)
    if name == "q4_0_ffn":
        return FfnQ4_0(g4, ctx, torch)
    if name == "q8_0_matvec":
        return MatvecQ8_0(g4, ctx, torch)
    if name == "q8_0_lm_head":
        return LmHeadQ8_0(g4, ctx, torch)
    if name == "q4_0_ffn_block":
        return FfnBlockQ4_0(g4, ctx, torch)
    if name == "q8_0_lm_head_cap":
        return LmHeadCapQ8_0(g4, ctx, torch)
    if name == "attention":
        return AttentionDecode(g4, ctx, torch, int(arg or 8192))
    if name == "q4_k_batched":
        return BatchedQ4_K(g4, ctx, torch, int(arg or 8))
    if name == "moe":
        return MoeQ4_K(g4, ctx, torch, int(arg or 1))
    if name in ("q5_k_matvec", "q6_k_matvec"):
        return MatvecKQuant(g4, ctx, torch, 13 if name == "q5_k_matvec" else 14)
    raise SystemExit("unknown workload %r" % spec)


def cpu_baseline(wl: Workload, seconds: float) -> dict:
    """Time the oracle (restated 512-bit Vector API path, OpenMP over rows like the
    reference's ForkJoin pool) on the host cores over a bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    threads = oracle.nthreads()
    wl.cpu_setup(oracle)
    if isinstance(wl, LmHeadQ8_0):
        rows = wl.cpu_sample_rows()
        n, t0 = 0, time.perf_counter()
        while True:
            wl.cpu_step_rows(rows)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 1000:
                break
        frac = rows / wl.V
        value = n * frac * wl.step_bytes / el / 1e9
        sample = "%d passes over %d of %d vocabulary rows (%.1f s)" % (n, rows, wl.V, el)
    else:
        n, t0 = 0, time.perf_counter()
        while True:
            wl.cpu_step()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 100000:
                break
        if wl.unit == "tokens/s":
            value = n * wl.tokens_per_step / el
        else:
            value = n * wl.step_bytes / el / 1e9
        sample = "%d steps of the same workload (%.1f s)" % (n, el)
    return {"value": round(value, 3), "unit": wl.unit, "cores": threads, "kind": "port", "sample": sample}


def _time_parts(wl, ctx, stream, torch, steps: int, use_graph: bool, capture) -> list:
    """Average launch time of each separately timed launch of a step: HIP events on
    the launch stream around back-to-back replays of a graph of that launch alone
    for steps 0 .. steps-1 -- the weight copies and routings the timed steps use,
    in a graph of the same length as the timed one -- replayed until at least 64
    launches are timed, after one untimed replay."""
    out = []
    reps = max(1, math.ceil(64 / steps))
    for name, nbytes, fn, tkey in wl.parts():
        g = None
        if use_graph:
            try:
                g = capture(lambda: [fn(i) for i in range(steps)])
            except Exception:
                g = None
                torch.cuda.synchronize()
        ctx.set_stream(stream.cuda_stream)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(reps):
            if g is not None:
                g.replay()
            else:
                for i in range(steps):
                    fn(i)
        ev1.record(stream)
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / (reps * steps)
        out.append({"kernel": name, "bytes_per_launch": nbytes, "avg_launch_us": round(us, 3),
                    "launches_timed": reps * steps, "traffic": TRAFFIC_BYTES.get(tkey)})
    return out


def run(spec: str, steps: int, warmup: int, cpu_seconds: float, use_graph: bool, ctx=None) -> dict:
    import torch
    import g4hip as g4
    if g4.device_count() == 0:
        raise SystemExit("bench.py needs a HIP device")
    torch.cuda.init()
    own_ctx = ctx is None
    if own_ctx:
        ctx = g4.Context(0)
    wl = make_workload(spec, g4, ctx, torch)
    stream = torch.cuda.Stream()

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            ctx.set_stream(stream.cuda_stream)
            fn()
        g.replay()
        torch.cuda.synchronize()
        return g

    with torch.cuda.stream(stream):
        ctx.set_stream(stream.cuda_stream)
        for i in range(warmup):
            wl.step(i)
        torch.cuda.synchronize()
        # the timed region is exactly `steps` steps, step i on weight copy / routing
        # i mod copies, captured as one graph (one replay: the graph's own launch
        # cost is spread over the steps as in a decode loop); the capture is
        # replayed once untimed first
        step_graph = None
        wl.set_steps(steps)
        if use_graph:
            try:
                step_graph = capture(lambda: [wl.step(i) for i in range(steps)])
            except Exception as e:
                print("graph capture unavailable (%s); timing eager launches" % str(e).splitlines()[0],
                      file=sys.stderr)
                step_graph = None
                torch.cuda.synchronize()
        # untimed replays of the step graph (about 20 ms of them): the GPU then runs
        # the timed steps warm, as a decode loop does (the first replays over a
        # large working set, such as the MoE experts, run up to 25% slower)
        if step_graph is not None:
            w0, n_warm = time.perf_counter(), 0
            while n_warm < 50 and (n_warm < 2 or time.perf_counter() - w0 < 0.02):
                step_graph.replay()
                torch.cuda.synchronize()
                n_warm += 1
        # a step's launches timed on their own where the dominant one is part of it
        parts = None if wl.dominant_is_step else _time_parts(wl, ctx, stream, torch, steps, use_graph, capture)
        ctx.set_stream(stream.cuda_stream)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        if step_graph is not None:
            step_graph.replay()
        else:
            for i in range(steps):
                wl.step(i)
        ev1.record(stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        if parts is None:
            # HIP events on the launch stream around the timed steps themselves
            us = ev0.elapsed_time(ev1) * 1e3 / steps
            parts = [{"kernel": wl.dominant_name, "bytes_per_launch": wl.dominant_bytes, "avg_launch_us": round(us, 3),
                      "launches_timed": steps, "traffic": TRAFFIC_BYTES.get(wl.name),
                      "timed": "HIP events around the timed region"}]
        graphed = step_graph is not None
        del step_graph
        ctx.set_stream(None)
    # the host-pointer entry point of the same step (copies in and out, synchronous;
    # not part of `value`): after a few untimed calls, the mean over whole passes
    host_us = None
    if wl.host_step is not None:
        for i in range(min(wl.copies, 4)):
            wl.host_step(i)
        n_host = wl.copies * max(1, math.ceil(16 / wl.copies))
        t0 = time.perf_counter()
        for i in range(n_host):
            wl.host_step(i)
        host_us = (time.perf_counter() - t0) / n_host * 1e6
    ms_per_step = elapsed * 1e3 / steps
    if wl.unit == "tokens/s":
        value = wl.tokens_per_step / (ms_per_step / 1e3)
        gbs_step = wl.step_bytes / (ms_per_step / 1e3) / 1e9
    else:
        value = wl.step_bytes / (ms_per_step / 1e3) / 1e9
        gbs_step = value
    for p in parts:
        gbs = p["bytes_per_launch"] / (p["avg_launch_us"] / 1e6) / 1e9
        p["achieved_gbs"] = round(gbs, 2)
        p["frac"] = round(gbs / HBM_PEAK_GBS, 4)
    dom = parts[0]
    kern_s = dom["avg_launch_us"] / 1e6
    achieved = wl.dominant_bytes / kern_s / 1e9
    if wl.bound == "mfma":
        tflops = wl.dominant_flops / kern_s / 1e12
        roofline = {"bound": "mfma", "achieved": round(tflops, 3), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 5), "traffic": TRAFFIC_BYTES.get(wl.name),
                    "hbm_gbs": round(achieved, 2), "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
                    "note": "useful flops 2*M*rows*cols; each fp32 product is three exact bf16 MFMA products"}
    else:
        roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_BYTES.get(wl.name)}
    roofline.update({"kernel": wl.dominant_name, "bytes_per_launch": wl.dominant_bytes,
                     "avg_launch_us": dom["avg_launch_us"], "launches_timed": dom["launches_timed"]})
    if len(parts) > 1:
        roofline["step_kernels"] = parts
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded GGUF blocks and activations (gemma4.kt_amd/synth.py)",
        "config": dict(wl.config(), graph=graphed, step_gbs=round(gbs_step, 2),
                       hbm_fraction=round(gbs_step / HBM_PEAK_GBS, 4)),
        # host-pointer calls (activations over PCIe each call), reported apart from value
        "host_pointer_call": None if host_us is None else {
            "us_per_step": round(host_us, 2),
            "value": round((wl.tokens_per_step if wl.unit == "tokens/s" else wl.step_bytes / 1e9) / (host_us / 1e6),
                           3),
            "unit": wl.unit},
        "roofline": roofline,
    }
    if cpu_seconds > 0 and not isinstance(wl, CopyCalibration):
        line["cpu_baseline"] = cpu_baseline(wl, cpu_seconds)
    del wl
    torch.cuda.synchronize()
    if own_ctx:
        ctx.close()
    return line


# Every other configuration the metric is quoted on, measured in the same run
# and reported in the default line's per_config object.
PER_CONFIG = ["q8_0_matvec", "q8_0_lm_head", "q4_k_batched:1", "q4_k_batched:8", "q4_k_batched:32",
              "q4_k_batched:64", "moe:1", "moe:16"]


def compact(line: dict) -> dict:
    """The per_config entry of one workload's line."""
    r = line["roofline"]
    c = {"workload": line["config"]["workload"], "value": line["value"], "unit": line["unit"],
         "ms_per_step": line["ms_per_step"], "steps": line["steps"], "step_gbs": line["config"]["step_gbs"],
         "hbm_fraction": line["config"]["hbm_fraction"],
         "roofline": {k: r[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel",
                                        "avg_launch_us") if k in r}}
    if "hbm_gbs" in r:
        c["roofline"]["hbm_gbs"], c["roofline"]["hbm_frac"] = r["hbm_gbs"], r["hbm_frac"]
    if "cpu_baseline" in line:
        c["cpu_baseline"] = line["cpu_baseline"]
    return c


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", default="q4_0_ffn", help="workload spec, or several separated by commas")
    ap.add_argument("--all", action="store_true", help="one JSON line per workload")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (0 = skip)")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    ap.add_argument("--no-per-config", action="store_true",
                    help="skip the other configurations in the default line's per_config object")
    ap.add_argument("--per-config-cpu-seconds", type=float, default=2.0,
                    help="CPU baseline sample length of each per_config entry")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    specs = args.workload.split(",")
    if args.all:
        specs = ["q4_0_ffn", "q8_0_matvec", "q8_0_lm_head", "q4_k_batched:1", "q4_k_batched:8",
                 "q4_k_batched:32", "q4_k_batched:64", "moe:1", "moe:16", "moe:128", "q5_k_matvec",
                 "q6_k_matvec", "q4_0_ffn_block", "q8_0_lm_head_cap", "attention:8192"]
    if args.steps < 1:
        raise SystemExit("--steps must be at least 1")
    default = not args.all and args.workload == "q4_0_ffn"
    for s in specs:
        line = run(s, args.steps, args.warmup, args.cpu_seconds, not args.eager)
        if default and not args.no_per_config:
            per = {}
            for spec in PER_CONFIG:
                print("per_config: %s" % spec, file=sys.stderr, flush=True)
                sub = run(spec, args.steps, args.warmup, args.per_config_cpu_seconds, not args.eager)
                per[sub["config"]["workload"]] = compact(sub)
            line["per_config"] = per
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
