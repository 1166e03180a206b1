#!/usr/bin/env python3
"""Benchmark: one decoder-layer decode step (M = 1 token) of the hot path on one MI355X.

A step is the three operators in layer order on one token: sliding_project_qkv (BASELINE
config 2) -> sliding_attention_output (config 1) -> decoder_feedforward with FP8 weights
(config 0, full FO/src/ops.rs contract incl. post-norm and layer scalar). Inputs are synthetic
(normal weights quantised to FP8 per channel), resident in HBM before timing.

MALL: all three weight sets fit the 256 MB Infinity Cache, so each operator cycles through
enough distinct weight copies (>= 512 MiB per operator) that no timed call re-reads cached
weights.

Timing: the K timed steps (--steps) are captured once in a HIP graph (as a decode loop replays
its captured layer); after W warm-up steps (--warmup, run as replays of the same graph) the graph
is replayed R >= 20 times back to back, with a HIP event on the replay stream (the stream the
kernels run on) between consecutive replays and synchronisations before the first and after the
last. Each replay is one run of exactly K steps; `value` is the median over the R replays of the
time per step, with p10 / p90 beside it. The operators are timed the same way (graphs of 40 calls).
Host-driven times (one Python/ctypes call per launch) are reported beside them.

Floor: an empty launch and a pure read of each operator's weight bytes (rotated past the MALL) at
the operator's launch shape, with the library's stream-read kernel, and the attainable read rate
of the device (1 GiB reads); the roofline's frac is also given against that attainable rate.

The per-operator list also times sliding_attention (the step between QKV and O, outside the
headline metric): one token over a full ring (1024 slots), caches rotated like the weights.

Prints one JSON line (stdout). `value` is microseconds per token for the step (lower is better);
`roofline` is for the dominant operator (the FFN); `cpu_baseline` times the CPU oracle (a C
restatement of the reference's algorithm) on this host's cores for a bounded sample.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--cpu-seconds 10]
    python bench.py --profile ffn|o|qkv [--steps 20]
    python bench.py --floor-shapes          # stream-read floor at several launch shapes
    python bench.py --vendor-gemm           # torch.matmul on the config-4 GEMM shapes

--profile runs one operator host-driven (one launch per call, no graph) over the rotating weight
copies, then one device-to-device copy of 256 MiB: the fixed workload the rocprofv3 counter runs
(FETCH_SIZE, WRITE_SIZE) use, the copy calibrating the counters against a known byte count.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "moa-workspace_amd"):
    sys.path.insert(0, str(p))

METRIC = "FFN/QKV/O decode µs/token at M=1 and % of HBM roofline (FP8 weights)"
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E spec
MALL_BYTES = 256 << 20
# Algorithmic bytes per call (weights + scales + operator-boundary vectors).
FATTN_PAGES = 8  # full-attention decode at position 4095: pages 0..7
BYTES = {"ffn": 177_116_176, "o": 15_775_232, "qkv": 31_523_848,
         # O then the FFN in one launch: both operators' bytes less the residual row between them,
         # which never goes to memory (one 7,680-byte write and one read)
         "o_ffn": 15_775_232 + 177_116_176 - 2 * 3840 * 2,
         # config 3, MXFP4 weights (E2M1 codes + E8M0 block-32 scales) at M = 1 and M = 16 rows: the
         # weights once, plus the rows' residual read and write, the two norm weights, the layer scalar
         "ffn_mxfp4": 94_003_200 + 2 * 3840 * 2 + 2 * 3840 * 2 + 16,
         # the reference's own FFN operand types (NVFP4: E2M1 codes, E4M3 block-16 scales, three f32
         # reciprocal global scales) on its run-0 inputs, M = 1
         "ffn_nvfp4": 3 * 29_491_200 + 3 * 3_686_400 + 3 * 4 + 2 * 3840 * 2 + 2 * 3840 * 2 + 16,
         "ffn_mxfp4_m16": 94_003_200 + 16 * 2 * 3840 * 2 + 2 * 3840 * 2 + 16,
         # the FP8 FFN at 16 rows: the M = 1 bytes plus 15 more residual rows read and written; the
         # same for the reference's NVFP4 operand types
         "ffn_m16": 177_116_176 + 15 * 2 * 3840 * 2,
         "ffn_nvfp4_m16": 3 * 29_491_200 + 3 * 3_686_400 + 3 * 4 + 16 * 2 * 3840 * 2 + 2 * 3840 * 2 + 16,
         # O at 16 rows (15 more input rows and residual rows read and written), and O then the
         # MXFP4 FFN on those 16 residual rows through one entry point (less the rows between them)
         "o_m16": 15_775_232 + 15 * (4096 * 2 + 2 * 3840 * 2),
         "o_ffn_mxfp4_m16": 15_775_232 + 15 * (4096 * 2 + 2 * 3840 * 2) + 94_003_200 + 16 * 2 * 3840 * 2
                            + 2 * 3840 * 2 + 16 - 16 * 2 * 3840 * 2,
         # sliding_attention, all 1024 slots valid: K and V caches + q + out + mask row
         "attn": 2 * 1024 * 8 * 256 * 2 + 2 * 4096 * 2 + 1024 * 4,
         # final_norm_and_logits: the bf16 lm_head (262144 x 3840) + input + norm weight + logits
         "logits": 262144 * 3840 * 2 + 2 * 3840 * 2 + 262144 * 2,
         # full-attention layers: QKV (Q 8192 + K 512 FP8 rows, bf16 scales; x, norms, cos/sin rows,
         # q_out, one K and one V slot), O with K = 8192 (weights, scales, x, sums, norm weight,
         # residual read + write), and the pages of a token at position 4095 (8 pages of K and V)
         "fqkv": 8704 * 3840 + 8704 * 2 + 3840 * 2 * 2 + 512 * 2 * 2 + 2 * 512 * 2 + 8192 * 2 + 2 * 512 * 2,
         "fo": 3840 * 8192 + 3840 * 2 + 8192 * 2 + 16 * 4 + 3840 * 2 + 2 * 3840 * 2,
         "fattn": FATTN_PAGES * 2 * 512 * 512 * 2 + FATTN_PAGES * (8192 * 2 + 512 * 4 + 8192 * 2 * 2 + 16 * 4 * 4),
         # the same pages in one fused call: K, V, q, masks, the state written once
         "fattn_fused": FATTN_PAGES * (2 * 512 * 512 * 2 + 512 * 4) + 8192 * 2 * 2 + 16 * 4 * 2,
         # the same at the cache's full 64 pages (position 32767)
         "fattn_fused64": 64 * (2 * 512 * 512 * 2 + 512 * 4) + 8192 * 2 * 2 + 16 * 4 * 2}
GRAPH_CALLS = 200  # calls per captured graph (as many as the headline step's K)
REPLAYS = 20  # timed replays per graph (median, p10, p90 over them)
# Config 4 (MFMA path): flops per token row; the MFMA runs bf16 x bf16 (FP8 weights widen exactly).
FLOPS_PER_ROW = {"qkv": 2 * 3840 * 8192, "o": 2 * 4096 * 3840, "ffn": 3 * 2 * 3840 * 15360}
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
MFMA_FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8
# Launch shapes (workgroups, threads) of the one-token kernels, for the floor measurements.
SHAPES = {"ffn": (240, 512), "o": (240, 512), "qkv": (256, 576)}
WEIGHT_BYTES = {"ffn": 3 * 15360 * 3840, "o": 3840 * 4096, "qkv": 8192 * 3840}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline sample length (0 = skip)")
    ap.add_argument("--ckpt-gib", type=float, default=1.0,
                    help="size of the synthetic checkpoint file the loader is timed on (0 = skip)")
    ap.add_argument("--chunk-rows", type=int, default=256,
                    help="rows of the config-4 layer chunk measured after the decode step (0 = skip)")
    ap.add_argument("--profile", choices=("ffn", "o", "qkv", "attn", "logits", "fqkv", "fattn", "fattn_fused", "fattn_fused64", "fo",
                                          "ffn_mxfp4", "ffn_mxfp4_m16", "ffn_m16", "ffn_nvfp4", "ffn_nvfp4_m16", "o_ffn", "o_m16", "o_ffn_mxfp4_m16",
                                          "chunk", "chunk_o_ffn", "floor"), default=None,
                    help="run one operator (or the config-4 layer chunk) host-driven for a counter profile, "
                         "then a 256 MiB copy")
    ap.add_argument("--floor-shapes", action="store_true",
                    help="only time the stream-read kernel graph-replayed at several launch shapes (an empty "
                         "launch and pure reads of O's and QKV's weight bytes); prints one JSON line")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only time torch.matmul (the vendor bf16 GEMM) on the chunk's four GEMM shapes with "
                         "bf16 weights, as a reference point for the MFMA path; prints one JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the hot path is a per-GPU kernel; "
                                   "run with --gpus 1 (multi-GPU sharding is a design note only)"}))
        return 2
    if args.vendor_gemm:
        return vendor_gemm(args.chunk_rows or 256)

    import numpy as np
    import torch

    from moa_amd import ops, synth

    torch.cuda.set_device(0)
    ops.init(0)
    if args.floor_shapes:
        sweep = floor_measure(torch, np, sweep=True)["sweep"]
        print(json.dumps({"floor_shapes_us": sweep, "timing": "graph-replayed, median over replays, launch included"}))
        return 0
    t0 = time.time()
    ffn = synth.cfg_ffn_fp8(0)
    o = synth.cfg_o(0)
    qkv = synth.cfg_qkv(0)
    att = synth.cfg_attention(0, M=1, pos=5000)
    log(f"synthesised inputs in {time.time() - t0:.1f}s")
    def dev(a):  # bf16 bits travel as int16 views (torch's uint16 support is partial)
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()

    def copies(nbytes):
        return max(2, math.ceil(2 * MALL_BYTES / nbytes) + 1)

    def replicate(d, keys, n):
        base = {k: dev(d[k]) for k in keys}
        return [base] + [{k: v.clone() for k, v in base.items()} for _ in range(n - 1)]

    nf, no, nq = copies(BYTES["ffn"]), copies(BYTES["o"]), copies(BYTES["qkv"])
    FW = replicate(ffn, ("up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
                         "down_weight_scale"), nf)
    OW = replicate(o, ("o_weight", "o_weight_scale"), no)
    QW = replicate(qkv, ("q_weight", "k_weight", "v_weight", "q_weight_scale", "k_weight_scale",
                         "v_weight_scale"), nq)
    na = copies(BYTES["attn"])
    AW = replicate(att, ("k_cache", "v_cache"), na)
    a_q, a_mask = dev(att["q"]), dev(att["mask"])
    a_out = torch.zeros(4096, dtype=torch.int16, device="cuda")
    # the lm_head (2 GB, one copy: it is 8x the MALL) is drawn on the device
    lg = synth.cfg_logits(0)
    lg_in, lg_rms, lg_w = dev(lg["input"]), dev(lg["rms_weight"]), synth.lm_head_device(0)
    lg_out = torch.zeros(synth.W, dtype=torch.int16, device="cuda")
    # full-attention layer operators: weights rotated like the others, the pages of position 4095
    fq = synth.cfg_full_qkv(0, pos=4095)
    fo = synth.cfg_full_o(0)
    fa = synth.cfg_full_attention(0, M=1, P=FATTN_PAGES)
    nfq, nfo, nfa = copies(BYTES["fqkv"]), copies(BYTES["fo"]), copies(BYTES["fattn"])
    FQW = replicate(fq, ("q_weight", "k_weight", "q_weight_scale", "k_weight_scale"), nfq)
    FOW = replicate(fo, ("o_weight", "o_weight_scale"), nfo)
    FAW = replicate(fa, ("k_pages", "v_pages"), nfa)
    fq_d = {k: dev(fq[k]) for k in ("x", "input_rms_weight", "q_rms_weight", "k_rms_weight", "cos", "sin",
                                    "k_cache", "v_cache")}
    fq_out = torch.zeros(8192, dtype=torch.int16, device="cuda")
    fq_kv = torch.tensor([fq["kv_offset"]], dtype=torch.int32, device="cuda")
    fq_ro = torch.tensor([fq["rope_offset"]], dtype=torch.int32, device="cuda")
    fo_d = {k: dev(fo[k]) for k in ("x", "running_sum", "post_attn_rms_weight", "residual")}
    fa_q, fa_masks = dev(fa["q"]), dev(fa["masks"])
    fa64 = synth.cfg_full_attention(1, M=1, P=64)
    nfa64 = copies(BYTES["fattn_fused64"])
    FAW64 = replicate(fa64, ("k_pages", "v_pages"), nfa64)
    fa64_q, fa64_masks = dev(fa64["q"]), dev(fa64["masks"])
    fa_max = torch.zeros(16, dtype=torch.float32, device="cuda")
    fa_sum = torch.zeros(16, dtype=torch.float32, device="cuda")
    fa_out = torch.zeros(8192, dtype=torch.int16, device="cuda")
    f_res, f_pre, f_post, f_ls = (dev(ffn[k]) for k in ("residual", "pre_ff_rms_weight", "post_ff_rms_weight",
                                                          "layer_scalar"))
    # config 3: MXFP4 weights, one row and 16 rows
    mx = synth.cfg_ffn_mxfp4(0, M=16)
    MXK = ("up_weight_packed", "gate_weight_packed", "down_weight_packed", "up_weight_scale", "gate_weight_scale",
           "down_weight_scale")
    nmx = copies(BYTES["ffn_mxfp4"])
    MXW = replicate(mx, MXK, nmx)
    mx_res16 = dev(mx["residual"])
    mx_res1 = mx_res16[:1].clone()
    nv = synth.ref_ffn_inputs(0)
    NVK = ("up_weight_packed", "gate_weight_packed", "down_weight_packed", "up_weight_scale", "gate_weight_scale",
           "down_weight_scale", "up_global_scale", "gate_global_scale", "down_global_scale")
    nnv = copies(BYTES["ffn_nvfp4"])
    NVW = replicate(nv, NVK, nnv)
    nv_res, nv_pre, nv_post, nv_ls = (dev(nv[k]) for k in ("residual", "pre_ff_rms_weight", "post_ff_rms_weight",
                                                             "layer_scalar"))
    o_x16 = dev(synth.bf16_normal("bench.o.x16", (16, 4096)))  # 16 attention rows for O at M = 16
    o_x, o_post, o_res = dev(o["x"]), dev(o["post_attn_rms_weight"]), dev(o["residual"])
    q = {k: dev(qkv[k]) for k in ("x", "input_rms_weight", "q_rms_weight", "k_rms_weight", "cos", "sin",
                                  "k_cache", "v_cache")}
    q_out = torch.zeros(4096, dtype=torch.int16, device="cuda")
    kv = torch.tensor([qkv["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([qkv["rope_offset"]], dtype=torch.int32, device="cuda")
    log(f"weight copies: ffn {nf}, o {no}, qkv {nq} "
        f"({(nf * BYTES['ffn'] + no * BYTES['o'] + nq * BYTES['qkv']) / 2**30:.2f} GiB)")

    # Config 4: one decoder-layer chunk of CM prefill rows (positions 0..CM-1) through the MFMA path,
    # on the same rotated FP8 weights; the O-projection's attention input is a seeded bf16 tensor.
    CM = args.chunk_rows
    if CM:
        ck = synth.cfg_layer_chunk(0, M=CM)
        c_x, c_attn = dev(ck["x"]), dev(ck["attn"])
        c_res = c_x.clone()  # the layer's residual stream: O adds into it, the FFN updates it
        c_cos, c_sin, c_kc, c_vc = (dev(ck[k]) for k in ("cos", "sin", "k_cache", "v_cache"))
        c_q = torch.zeros(CM * 4096, dtype=torch.int16, device="cuda")
        c_kv = torch.tensor([ck["kv_offset"]], dtype=torch.int32, device="cuda")
        c_ro = torch.tensor([ck["rope_offset"]], dtype=torch.int32, device="cuda")

    def run_cqkv(i):
        w = QW[i % nq]
        ops.sliding_project_qkv(c_x, w["q_weight"], w["k_weight"], w["v_weight"], w["q_weight_scale"],
                                w["k_weight_scale"], w["v_weight_scale"], q["input_rms_weight"], q["q_rms_weight"],
                                q["k_rms_weight"], c_kv, c_ro, c_cos, c_sin, c_kc, c_vc, c_q)

    def run_co(i):
        w = OW[i % no]
        ops.sliding_attention_output(c_attn, o_post, w["o_weight"], w["o_weight_scale"], c_res)

    def run_cffn(i):
        w = FW[i % nf]
        ops.decoder_feedforward_fp8(c_res, f_pre, w["up_weight"], w["gate_weight"], w["down_weight"],
                                    w["up_weight_scale"], w["gate_weight_scale"], w["down_weight_scale"],
                                    f_post, f_ls)

    def run_layer(i):
        run_cqkv(i)
        run_co(i)
        run_cffn(i)

    def run_layer_o_ffn(i):
        # the same layer with O and the FFN through one entry point (O's post rows also write the
        # FFN's normalised input)
        run_cqkv(i)
        v, w = OW[i % no], FW[i % nf]
        ops.sliding_attention_output_feedforward_fp8(
            c_attn, o_post, v["o_weight"], v["o_weight_scale"], c_res, f_pre, w["up_weight"], w["gate_weight"],
            w["down_weight"], w["up_weight_scale"], w["gate_weight_scale"], w["down_weight_scale"], f_post, f_ls)

    if CM:
        c_res_mx = dev(synth.bf16_normal("cfg4.mxfp4.residual", (CM, 3840)))

    def run_cffn_mxfp4(i):
        w = MXW[i % nmx]
        ops.decoder_feedforward_mxfp4(c_res_mx, f_pre, *[w[k] for k in MXK], f_post, f_ls)

    def run_ffn(i):
        w = FW[i % nf]
        ops.decoder_feedforward_fp8(f_res, f_pre, w["up_weight"], w["gate_weight"], w["down_weight"],
                                    w["up_weight_scale"], w["gate_weight_scale"], w["down_weight_scale"],
                                    f_post, f_ls)

    def run_ffn_mxfp4(i, res=None):
        w = MXW[i % nmx]
        ops.decoder_feedforward_mxfp4(mx_res1 if res is None else res, f_pre, *[w[k] for k in MXK], f_post, f_ls)

    def run_ffn_nvfp4(i):
        w = NVW[i % nnv]
        ops.decoder_feedforward(nv_res, nv_pre, *[w[k] for k in NVK], nv_post, nv_ls)

    def run_ffn_mxfp4_m16(i):
        run_ffn_mxfp4(i, mx_res16)

    def run_ffn_nvfp4_m16(i):
        w = NVW[i % nnv]
        ops.decoder_feedforward(mx_res16, nv_pre, *[w[k] for k in NVK], nv_post, nv_ls)

    def run_ffn_m16(i):
        w = FW[i % nf]
        ops.decoder_feedforward_fp8(mx_res16, f_pre, w["up_weight"], w["gate_weight"], w["down_weight"],
                                    w["up_weight_scale"], w["gate_weight_scale"], w["down_weight_scale"],
                                    f_post, f_ls)

    def run_o(i):
        w = OW[i % no]
        ops.sliding_attention_output(o_x, o_post, w["o_weight"], w["o_weight_scale"], o_res)

    def run_o_m16(i):
        w = OW[i % no]
        ops.sliding_attention_output(o_x16, o_post, w["o_weight"], w["o_weight_scale"], mx_res16)

    def run_o_ffn_mxfp4_m16(i):
        # 16 rows of O then the MXFP4 FFN through one entry point (the rows path: O's post rows
        # also write the FFN's normalised input)
        v, w = OW[i % no], MXW[i % nmx]
        ops.sliding_attention_output_feedforward_mxfp4(o_x16, o_post, v["o_weight"], v["o_weight_scale"], mx_res16,
                                                       f_pre, *[w[k] for k in MXK], f_post, f_ls)

    def run_o_ffn(i):
        v, w = OW[i % no], FW[i % nf]
        ops.sliding_attention_output_feedforward_fp8(
            o_x, o_post, v["o_weight"], v["o_weight_scale"], f_res, f_pre, w["up_weight"], w["gate_weight"],
            w["down_weight"], w["up_weight_scale"], w["gate_weight_scale"], w["down_weight_scale"], f_post, f_ls)

    def run_qkv(i):
        w = QW[i % nq]
        ops.sliding_project_qkv(q["x"], w["q_weight"], w["k_weight"], w["v_weight"], w["q_weight_scale"],
                                w["k_weight_scale"], w["v_weight_scale"], q["input_rms_weight"], q["q_rms_weight"],
                                q["k_rms_weight"], kv, ro, q["cos"], q["sin"], q["k_cache"], q["v_cache"], q_out)

    def run_attn(i):
        w = AW[i % na]
        ops.sliding_attention(a_q, w["k_cache"], w["v_cache"], a_mask, a_out)

    def run_qkv_then_attn(i):
        # QKV writes its slot into the attention's rotated caches and the attention reads them
        w, c = QW[i % nq], AW[i % na]
        ops.sliding_project_qkv(q["x"], w["q_weight"], w["k_weight"], w["v_weight"], w["q_weight_scale"],
                                w["k_weight_scale"], w["v_weight_scale"], q["input_rms_weight"], q["q_rms_weight"],
                                q["k_rms_weight"], kv, ro, q["cos"], q["sin"], c["k_cache"], c["v_cache"], q_out)
        ops.sliding_attention(q_out, c["k_cache"], c["v_cache"], a_mask, a_out)

    def run_fqkv(i):
        w = FQW[i % nfq]
        ops.full_project_qkv(fq_d["x"], w["q_weight"], w["k_weight"], w["q_weight_scale"], w["k_weight_scale"],
                             fq_d["input_rms_weight"], fq_d["q_rms_weight"], fq_d["k_rms_weight"], fq_kv, fq_ro,
                             fq_d["cos"], fq_d["sin"], fq_d["k_cache"], fq_d["v_cache"], fq_out)

    def run_fo(i):
        w = FOW[i % nfo]
        ops.full_attention_output(fo_d["x"], fo_d["running_sum"], fo_d["post_attn_rms_weight"], w["o_weight"],
                                  w["o_weight_scale"], fo_d["residual"])

    def run_fattn(i):
        w = FAW[i % nfa]
        for pg in range(FATTN_PAGES):
            fn = ops.full_attention_first_page if pg == 0 else ops.full_attention_page
            fn(fa_q, w["k_pages"][pg], w["v_pages"][pg], fa_masks[pg], fa_max, fa_sum, fa_out)

    def run_fattn_fused(i):
        w = FAW[i % nfa]
        ops.full_attention(fa_q, w["k_pages"], w["v_pages"], fa_masks, fa_max, fa_sum, fa_out)

    def run_fattn_fused64(i):
        w = FAW64[i % nfa64]
        ops.full_attention(fa64_q, w["k_pages"], w["v_pages"], fa64_masks, fa_max, fa_sum, fa_out)

    def run_logits(i):
        ops.final_norm_and_logits(lg_in, lg_rms, lg_w, lg_out)

    def run_step(i):
        run_qkv(i)
        run_o(i)
        run_ffn(i)

    def run_layer_calls(i):  # the sliding layer's decode step as the runtime calls it: four operators
        run_qkv_then_attn(i)
        run_o(i)
        run_ffn(i)

    def run_layer_fused(i):  # the same with O and the FFN in one launch: three launches
        run_qkv_then_attn(i)
        run_o_ffn(i)

    def run_step_fused(i):
        run_qkv(i)
        run_o_ffn(i)

    def timed(fn, steps, warmup):
        """Host-driven: one library call per launch (includes Python/ctypes submission)."""
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            fn(warmup + i)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps  # ms per call

    def graph_stats(fn, calls=GRAPH_CALLS, warmup=GRAPH_CALLS, replays=REPLAYS):
        """Graph-driven: `calls` consecutive calls (cycling the weight copies) captured once in a
        HIP graph; warm-up replays covering `warmup` calls, then `replays` replays back to back with
        an event between consecutive ones on the replay stream. Returns the median, p10 and p90 of
        ms per call over the replays. At least two warm-up replays: the first replays after a
        capture run slow (measured on the FFN with 40-call graphs: the first 8 of 20 replays 2-5 %
        slower than the rest; with 200-call graphs only the first)."""
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(calls):
                fn(i)
        for _ in range(max(2, math.ceil(warmup / calls))):
            g.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
        ev[0].record()
        for r in range(replays):
            g.replay()
            ev[r + 1].record()
        torch.cuda.synchronize()
        per = np.array([ev[r].elapsed_time(ev[r + 1]) / calls for r in range(replays)])
        del g
        return float(np.median(per)), float(np.percentile(per, 10)), float(np.percentile(per, 90))

    if args.profile == "floor":
        floor_profile(torch, args.steps)
        return 0
    if args.profile:
        fn = {"ffn": run_ffn, "o": run_o, "qkv": run_qkv, "attn": run_attn, "logits": run_logits,
              "fqkv": run_fqkv, "fattn": run_fattn, "fattn_fused": run_fattn_fused,
              "fattn_fused64": run_fattn_fused64, "fo": run_fo, "ffn_mxfp4": run_ffn_mxfp4,
              "ffn_mxfp4_m16": run_ffn_mxfp4_m16, "ffn_m16": run_ffn_m16, "ffn_nvfp4_m16": run_ffn_nvfp4_m16,
              "chunk": run_layer,
              "chunk_o_ffn": run_layer_o_ffn,
              "o_ffn": run_o_ffn, "o_m16": run_o_m16, "o_ffn_mxfp4_m16": run_o_ffn_mxfp4_m16,
              "ffn_nvfp4": run_ffn_nvfp4}[args.profile]
        for i in range(args.steps):
            fn(i)
        torch.cuda.synchronize()
        src = torch.empty(128 << 20, dtype=torch.int16, device="cuda")  # 256 MiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"profile: {args.steps} x {args.profile}, then a copy of {src.numel() * 2} bytes")
        assert ops.device_errors() == 0
        return 0

    floor = floor_measure(torch, np)

    per_op = {}
    for name, fn in (("qkv", run_qkv), ("o", run_o), ("ffn", run_ffn), ("o_ffn", run_o_ffn), ("ffn_mxfp4", run_ffn_mxfp4),
                     ("ffn_mxfp4_m16", run_ffn_mxfp4_m16), ("ffn_m16", run_ffn_m16), ("ffn_nvfp4", run_ffn_nvfp4),
                     ("ffn_nvfp4_m16", run_ffn_nvfp4_m16),
                     ("o_m16", run_o_m16),
                     ("o_ffn_mxfp4_m16", run_o_ffn_mxfp4_m16),
                     ("attn", run_attn), ("logits", run_logits),
                     ("fqkv", run_fqkv), ("fattn", run_fattn), ("fattn_fused", run_fattn_fused),
                     ("fattn_fused64", run_fattn_fused64), ("fo", run_fo)):
        ms, p10, p90 = graph_stats(fn, replays=5 if name == "logits" else REPLAYS)
        ms_host = timed(fn, min(args.steps, 50), 5)
        gbps = BYTES[name] / (ms * 1e-3) / 1e9
        per_op[name] = {"us": round(ms * 1e3, 3), "us_p10": round(p10 * 1e3, 3), "us_p90": round(p90 * 1e3, 3),
                        "GBps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
                        "frac_attainable": round(gbps / floor["attainable_read_GBps"], 4),
                        "bytes": BYTES[name], "us_host_driven": round(ms_host * 1e3, 3)}
        log(f"{name:13} {ms * 1e3:9.2f} us [p10 {p10 * 1e3:.2f}, p90 {p90 * 1e3:.2f}]  {gbps:8.1f} GB/s  "
            f"{100 * gbps / HBM_PEAK_GBPS:5.1f}% of 8 TB/s   (host-driven {ms_host * 1e3:.2f} us)")

    # the headline: a graph of exactly K steps, replayed REPLAYS times after the warm-up
    ms_step, step_p10, step_p90 = graph_stats(run_step, calls=args.steps, warmup=max(args.warmup, 1))
    ms_step_host = timed(run_step, min(args.steps, 50), 5)
    log(f"step {ms_step * 1e3:9.2f} us/token [p10 {step_p10 * 1e3:.2f}, p90 {step_p90 * 1e3:.2f}]   "
        f"(host-driven {ms_step_host * 1e3:.2f} us)")
    # the same step with O and the FFN in one launch (moa_sliding_attention_output_feedforward_fp8)
    ms_fstep, fstep_p10, fstep_p90 = graph_stats(run_step_fused, calls=args.steps, warmup=max(args.warmup, 1))
    log(f"step, O->FFN fused {ms_fstep * 1e3:9.2f} us/token [p10 {fstep_p10 * 1e3:.2f}, p90 {fstep_p90 * 1e3:.2f}]")
    # the whole sliding-layer step (attention included): four calls, and three launches
    ms_lc, lc_p10, lc_p90 = graph_stats(run_layer_calls, calls=args.steps, warmup=max(args.warmup, 1))
    ms_lf, lf_p10, lf_p90 = graph_stats(run_layer_fused, calls=args.steps, warmup=max(args.warmup, 1))
    log(f"layer step: four calls {ms_lc * 1e3:9.2f} us, three launches {ms_lf * 1e3:9.2f} us")

    chunk = None
    if CM:
        chunk = {"rows": CM, "peak_TFLOPs": MFMA_BF16_PEAK_TFLOPS, "peak_fp8_TFLOPs": MFMA_FP8_PEAK_TFLOPS, "ops": {}}
        for name, fn in (("qkv", run_cqkv), ("o", run_co), ("ffn", run_cffn), ("layer", run_layer),
                         ("layer_o_ffn", run_layer_o_ffn), ("ffn_mxfp4", run_cffn_mxfp4)):
            ms, p10, p90 = graph_stats(fn, calls=8, warmup=8, replays=10)
            flops = CM * (sum(FLOPS_PER_ROW.values()) if name.startswith("layer") else FLOPS_PER_ROW[name.split("_")[0]])
            tf = flops / (ms * 1e-3) / 1e12
            chunk["ops"][name] = {"us": round(ms * 1e3, 2), "us_p10": round(p10 * 1e3, 2), "us_p90": round(p90 * 1e3, 2),
                                  "us_per_token": round(ms * 1e3 / CM, 4), "TFLOPs": round(tf, 1),
                                  "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                                  "frac_fp8_peak": round(tf / MFMA_FP8_PEAK_TFLOPS, 4), "flops": flops}
            log(f"chunk M={CM} {name:5} {ms * 1e3:9.2f} us  {tf:7.1f} TFLOP/s  "
                f"{100 * tf / MFMA_BF16_PEAK_TFLOPS:5.1f}% of bf16 / {100 * tf / MFMA_FP8_PEAK_TFLOPS:5.1f}% of fp8 peak")

    ckpt = ckpt_measure(args.ckpt_gib) if args.ckpt_gib > 0 else None
    if ckpt:
        ckpt["file_GiB"] = args.ckpt_gib

    # attainable HBM bandwidth: device-to-device copy of 2 GiB (read + write)
    big = torch.empty(1 << 30, dtype=torch.int16, device="cuda")
    dst = torch.empty_like(big)
    cp_ms = timed(lambda i: dst.copy_(big), 10, 3)
    copy_gbps = 2 * big.numel() * 2 / (cp_ms * 1e-3) / 1e9
    del big, dst
    assert ops.device_errors() == 0

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(ffn, o, qkv, args.cpu_seconds)
        lm_rows = lg_w[:LOGITS_CPU_ROWS].cpu().numpy().view(np.uint16)
        for name, us, sample in cpu_next_ops(att, lg, lm_rows, fq, fa, fo):
            per_op[name]["cpu_us"] = round(us, 1)
            per_op[name]["cpu_sample"] = sample

    f = per_op["ffn"]
    # HBM bytes per FFN launch from the committed counter profile (FETCH_SIZE / WRITE_SIZE runs,
    # calibrated against a copy of known size); null when the profile is absent.
    traffic = None
    tpath = ROOT / "profiles" / "hbm_traffic_m1.json"
    if tpath.exists():
        traffic = json.loads(tpath.read_text()).get("ffn_fused_kernel", {}).get("traffic_bytes")
    line = {
        "metric": METRIC, "value": round(ms_step * 1e3, 3), "unit": "us/token", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "timing": {"steps_per_replay": args.steps, "replays": REPLAYS, "steps_timed_total": args.steps * REPLAYS,
                   "value_is": "median over replays of us per step", "us_p10": round(step_p10 * 1e3, 3),
                   "us_p90": round(step_p90 * 1e3, 3)},
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8e4m3 weights x bf16 activations, f32 accumulate", "data": "synthetic",
        "config": {"workload": "decode step, M=1: sliding_project_qkv (cfg2) + sliding_attention_output (cfg1) "
                               "+ decoder_feedforward FP8 (cfg0); weights rotated over >=512 MiB per operator",
                   "hidden": 3840, "intermediate": 15360, "tokens_per_step": 1},
        "roofline": {"bound": "hbm", "kernel": "decoder_feedforward_fp8 (ffn_fused_kernel, one launch)",
                     "achieved": f["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": f["frac"],
                     "attainable": floor["attainable_read_GBps"], "frac_attainable": f["frac_attainable"],
                     "algorithmic_bytes": BYTES["ffn"], "avg_us": f["us"], "traffic": traffic,
                     "traffic_source": "profiles/hbm_traffic_m1.md" if traffic else None},
        "ops": per_op,
        "step_o_ffn_fused": {"us": round(ms_fstep * 1e3, 3), "us_p10": round(fstep_p10 * 1e3, 3),
                             "us_p90": round(fstep_p90 * 1e3, 3),
                             "workload": "sliding_project_qkv (cfg2) + sliding_attention_output_feedforward_fp8 "
                                         "(cfg1 then cfg0, one launch)"},
        "layer_step": {"us_four_calls": round(ms_lc * 1e3, 3), "us_four_calls_p90": round(lc_p90 * 1e3, 3),
                       "us_three_launches": round(ms_lf * 1e3, 3), "us_three_launches_p90": round(lf_p90 * 1e3, 3),
                       "workload": "the sliding layer's decode step with its attention (pos 5000, all 1024 "
                                   "slots): sliding_project_qkv, sliding_attention, sliding_attention_output, "
                                   "decoder_feedforward_fp8 as four calls, and with the last two through "
                                   "sliding_attention_output_feedforward_fp8 (one launch)"},
        "floor": floor,
        "us_per_token_host_driven": round(ms_step_host * 1e3, 3),
        "hbm_copy_GBps": round(copy_gbps, 1),
        "cpu_baseline": cpu,
        "checkpoint_load": ckpt,
        "chunk": chunk,
    }
    print(json.dumps(line), flush=True)
    return 0


def ckpt_measure(gib: float = 1.0):
    """The checkpoint reader (moa_ckpt_load_bf16) on a synthetic one-tensor safetensors file of
    `gib` GiB, already in the page cache: host-to-device GB/s, median of 3 loads, beside a plain
    pinned-memory copy of the same size (torch) as the link's attainable rate."""
    import tempfile

    import numpy as np
    import torch

    from moa_amd import checkpoint

    rows = int(gib * 2**30) // (3840 * 2)
    nbytes = rows * 3840 * 2
    hdr = json.dumps({"t": {"dtype": "BF16", "shape": [rows, 3840], "data_offsets": [0, nbytes]}}).encode()
    hdr += b" " * (-len(hdr) % 8)
    d = tempfile.mkdtemp(dir=os.environ.get("TMPDIR"))
    path = os.path.join(d, "model.safetensors")
    chunk = np.random.default_rng(0).integers(0, 1 << 16, size=(64 << 20) // 2, dtype=np.uint16).tobytes()
    with open(path, "wb") as f:
        f.write(len(hdr).to_bytes(8, "little") + hdr)
        left = nbytes
        while left:
            f.write(chunk[: min(left, len(chunk))])
            left -= min(left, len(chunk))
    try:
        times = []
        with checkpoint.Checkpoint(path) as ck:
            for _ in range(4):
                torch.cuda.synchronize()
                t = time.perf_counter()
                x = ck.load_bf16("t", (rows, 3840))
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t)
                del x
        pinned = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        ptimes = []
        for _ in range(3):
            torch.cuda.synchronize()
            t = time.perf_counter()
            dst.copy_(pinned, non_blocking=True)
            torch.cuda.synchronize()
            ptimes.append(time.perf_counter() - t)
        del pinned, dst
    finally:
        os.remove(path)
        os.rmdir(d)
    gbps = nbytes / float(np.median(times[1:])) / 1e9
    link = nbytes / float(np.median(ptimes)) / 1e9
    log(f"checkpoint load {gbps:7.1f} GB/s (pinned host-to-device copy {link:.1f} GB/s)")
    return {"GBps": round(gbps, 1), "pinned_copy_GBps": round(link, 1), "bytes": nbytes}


FLOOR_SWEEP_SHAPES = ((240, 256), (240, 512), (256, 256), (256, 576), (256, 1024))


def floor_measure(torch, np, sweep: bool = False):
    """The library's stream-read kernel (moa_bench_stream_read): the device's attainable read rate
    (1 GiB per launch, best of three launch shapes), and per one-token operator an empty launch and
    a pure read of its weight bytes at its launch shape, the windows rotated over 1 GiB so no
    launch reads from the MALL. Graph-replayed like the operators. With sweep, only the empty
    launch and the reads of O's and QKV's bytes at each of FLOOR_SWEEP_SHAPES (out["sweep"])."""
    import ctypes as C

    from moa_amd import _lib

    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def read(nbytes, shape, rotate=True):
        span = buf.numel() - nbytes
        def fn(i):
            off = ((i * nbytes) % span) // 256 * 256 if rotate and nbytes else 0
            _lib.call("moa_bench_stream_read", C.c_void_p(buf.data_ptr() + off), C.c_uint64(nbytes), shape[0],
                      shape[1], C.c_void_p(sink.data_ptr()), stream())
        return fn

    def stats(fn, calls=GRAPH_CALLS):
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(calls):
                fn(i)
        g.replay()
        g.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(REPLAYS + 1)]
        ev[0].record()
        for r in range(REPLAYS):
            g.replay()
            ev[r + 1].record()
        torch.cuda.synchronize()
        per = np.array([ev[r].elapsed_time(ev[r + 1]) / calls for r in range(REPLAYS)])
        return float(np.median(per)) * 1e3  # us

    if sweep:
        table = {}
        for label, nbytes in (("empty", 0), ("o", WEIGHT_BYTES["o"]), ("qkv", WEIGHT_BYTES["qkv"])):
            for shape in FLOOR_SWEEP_SHAPES:
                us = stats(read(nbytes, shape))
                table[f"{label} {shape[0]}x{shape[1]}"] = round(us, 3)
                log(f"floor sweep {label:5} {shape}: {us:.2f} us")
        del buf
        return {"sweep": table}
    out = {"attainable_shapes": {}}
    for shape in ((1024, 512), (512, 1024), (2048, 256)):
        us = stats(read(buf.numel(), shape, rotate=False), calls=8)
        out["attainable_shapes"][f"{shape[0]}x{shape[1]}"] = round(buf.numel() / (us * 1e-6) / 1e9, 1)
    out["attainable_read_GBps"] = max(out["attainable_shapes"].values())
    for name, shape in SHAPES.items():
        empty = stats(read(0, shape))
        full = stats(read(WEIGHT_BYTES[name], shape))
        out[name] = {"shape": list(shape), "empty_us": round(empty, 3), "read_us": round(full, 3),
                     "read_bytes": WEIGHT_BYTES[name], "read_GBps": round(WEIGHT_BYTES[name] / (full * 1e-6) / 1e9, 1)}
        log(f"floor {name:4} {shape}: empty launch {empty:.2f} us, read of {WEIGHT_BYTES[name]} B {full:.2f} us")
    log(f"attainable read rate {out['attainable_read_GBps']:.1f} GB/s ({out['attainable_shapes']})")
    del buf
    return out


FLOOR_SEQUENCE = [  # (label, bytes, workgroups, threads) in dispatch order for --profile floor
    ("empty o/ffn shape", 0, 240, 512), ("empty qkv shape", 0, 256, 576),
    ("read o weights", WEIGHT_BYTES["o"], 240, 512), ("read qkv weights", WEIGHT_BYTES["qkv"], 256, 576),
    ("read ffn weights", WEIGHT_BYTES["ffn"], 240, 512), ("read 1 GiB", 1 << 30, 1024, 512)]


def vendor_gemm(rows: int) -> int:
    """The vendor bf16 GEMM (torch.matmul, which calls hipBLASLt) on the config-4 chunk's GEMM shapes:
    X [rows, K] bf16 times W [N, K]^T with bf16 weights (twice the bytes of FP8), copies rotated over
    >= 512 MiB, 20 calls per HIP graph, median of 10 replays. Nothing of the library runs here: it
    is a reference point for what a library GEMM reaches on these shapes."""
    import numpy as np
    import torch

    torch.cuda.set_device(0)
    out = {}
    for name, n, k in (("up+gate", 2 * 15360, 3840), ("down", 3840, 15360), ("qkv", 8192, 3840), ("o", 3840, 4096)):
        x = torch.randn(rows, k, device="cuda", dtype=torch.bfloat16)
        ws = [torch.randn(n, k, device="cuda", dtype=torch.bfloat16) for _ in range(max(2, -(-(512 << 20) // (n * k * 2))))]
        for i in range(3):
            x @ ws[i % len(ws)].t()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(20):
                x @ ws[i % len(ws)].t()
        g.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(11)]
        ev[0].record()
        for r in range(10):
            g.replay()
            ev[r + 1].record()
        torch.cuda.synchronize()
        us = float(np.median([ev[r].elapsed_time(ev[r + 1]) / 20 * 1e3 for r in range(10)]))
        tf = 2 * rows * n * k / us / 1e6
        out[name] = {"N": n, "K": k, "us": round(us, 2), "TFLOPs": round(tf, 1), "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
        log(f"vendor bf16 GEMM {name:8} M={rows} N={n} K={k}: {us:8.2f} us  {tf:7.1f} TFLOP/s")
        del ws, g
    print(json.dumps({"vendor_gemm": {"rows": rows, "weights": "bf16", "ops": out}}))
    return 0


def floor_profile(torch, steps: int) -> None:
    """Host-driven stream-read launches for a kernel trace: `steps` launches of each FLOOR_SEQUENCE
    entry in order (reads rotated over a 1 GiB buffer, 1 GiB reads from a second one), with a
    synchronisation between entries; then the 256 MiB copy of the other profiles."""
    import ctypes as C

    from moa_amd import _lib

    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for label, nbytes, wg, thr in FLOOR_SEQUENCE:
        for i in range(steps):
            if nbytes == 1 << 30:
                ptr = big.data_ptr()
            else:
                span = buf.numel() - nbytes
                ptr = buf.data_ptr() + (((i * nbytes) % span) // 256 * 256 if nbytes else 0)
            _lib.call("moa_bench_stream_read", C.c_void_p(ptr), C.c_uint64(nbytes), wg, thr, C.c_void_p(sink.data_ptr()), st)
        torch.cuda.synchronize()
        log(f"profile floor: {steps} x {label} ({nbytes} B, {wg} x {thr})")


LOGITS_CPU_ROWS = 16384  # vocabulary rows of the CPU logits sample (1/16 of the vocabulary)


def cpu_next_ops(att, lg, lm_rows, fq, fa, fo, seconds: float = 1.0):
    """The CPU oracle on the next-row operators' bench inputs: median wall time per call, about a
    second of calls each (16 OpenMP threads). Logits: a sample of LOGITS_CPU_ROWS vocabulary rows,
    scaled to the full 262144."""
    import numpy as np

    from oracle import oracle as O

    def med(fn):
        fn()
        times, t_end = [], time.time() + seconds
        while time.time() < t_end or len(times) < 3:
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
        return float(np.median(times)) * 1e6

    kp, vp, qo = fq["k_cache"].copy(), fq["v_cache"].copy(), np.zeros(8192, np.uint16)
    unb = lambda b: (b.astype(np.uint32) << 16).view(np.float32)
    res = fo["residual"].copy()
    out = [
        ("attn", med(lambda: O.sliding_attention(att["q"], att["k_cache"], att["v_cache"], att["mask"])),
         "one call (M=1, 1024 slots)"),
        ("logits", med(lambda: O.final_norm_and_logits(lg["input"], lg["rms_weight"], lm_rows)) * (262144 / len(lm_rows)),
         f"{len(lm_rows)} vocabulary rows, scaled to 262144"),
        ("fqkv", med(lambda: O.full_project_qkv(fq["x"], fq["q_weight"], fq["k_weight"], unb(fq["q_weight_scale"]),
                                                unb(fq["k_weight_scale"]), fq["input_rms_weight"], fq["q_rms_weight"],
                                                fq["k_rms_weight"], fq["kv_offset"], fq["rope_offset"], fq["cos"],
                                                fq["sin"], kp, vp, qo)), "one call (M=1)"),
        ("fattn_fused", med(lambda: O.full_attention_pages(fa["q"], fa["k_pages"], fa["v_pages"], fa["masks"])),
         f"one call ({fa['masks'].shape[0]} pages)"),
        ("fo", med(lambda: O.full_attention_output(fo["x"], fo["running_sum"], fo["post_attn_rms_weight"],
                                                   fo["o_weight"], unb(fo["o_weight_scale"]), res)), "one call (M=1)"),
    ]
    for name, us, _ in out:
        log(f"cpu oracle {name:11} {us:10.1f} us")
    return out


def cpu_baseline(ffn, o, qkv, seconds: float):
    """The CPU oracle (C restatement of the reference's algorithm) on this host, same inputs."""
    import numpy as np

    from oracle import oracle as O

    avail = len(os.sched_getaffinity(0))
    cores = min(avail, int(os.environ.get("OMP_NUM_THREADS") or avail))  # the box's CPU share
    O.set_threads(cores)
    w = O.ffn_weights(O.FFN_FP8, ffn["up_weight"], ffn["gate_weight"], ffn["down_weight"], ffn["up_weight_scale"],
                      ffn["gate_weight_scale"], ffn["down_weight_scale"])
    kc, vc, qo = qkv["k_cache"].copy(), qkv["v_cache"].copy(), np.zeros(4096, np.uint16)
    r_o, r_f = o["residual"].copy(), ffn["residual"].copy()

    def step():
        O.sliding_project_qkv(qkv["x"], qkv["q_weight"], qkv["k_weight"], qkv["v_weight"], qkv["q_weight_scale"],
                              qkv["k_weight_scale"], qkv["v_weight_scale"], qkv["input_rms_weight"],
                              qkv["q_rms_weight"], qkv["k_rms_weight"], qkv["kv_offset"], qkv["rope_offset"],
                              qkv["cos"], qkv["sin"], kc, vc, qo)
        O.sliding_attention_output(o["x"], o["post_attn_rms_weight"], o["o_weight"], o["o_weight_scale"], r_o)
        O.decoder_feedforward(r_f, ffn["pre_ff_rms_weight"], w, ffn["post_ff_rms_weight"], ffn["layer_scalar"])

    def median_us(n_min, budget):
        step()  # warm-up
        times = []
        t_end = time.time() + budget
        while time.time() < t_end or len(times) < n_min:
            t = time.perf_counter()
            step()
            times.append(time.perf_counter() - t)
        return float(np.median(times)) * 1e6, len(times)

    us, n = median_us(20, seconds)
    O.set_threads(1)
    us1, n1 = median_us(20, 0.0)
    O.set_threads(cores)
    model = "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    log(f"cpu oracle {us:9.1f} us/token on {cores} threads ({n} steps), {us1:.1f} us on 1 thread ({n1} steps); "
        f"{avail} cores available, {model}")
    return {"value": round(us, 1), "unit": "us/token", "cores": cores, "kind": "port",
            "cores_available": avail, "cpu_model": model, "one_thread_value": round(us1, 1),
            "sample": f"{n} decode steps (M=1, cfg0+cfg1+cfg2), median, OpenMP {cores} threads; "
                      f"1 thread: median of {n1} steps"}


if __name__ == "__main__":
    sys.exit(main())
