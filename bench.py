#!/usr/bin/env python3
"""Benchmark of the kquant_amd hot path on one MI355X.

Prints ONE JSON line.  The headline (``value``) is benchmark configuration 2's
MXFP8 weight quantization: W [12288, 7168] bf16 -> E4M3 codes + E8M0 scales;
a step is one quantization of that weight, inputs resident in HBM.  The
second half of the metric, the MXFP4 expert GEMM TFLOP/s, is the configuration
3 grouped MoE prefill (``moe_prefill``).  Every other configuration is
reported beside it with its own roofline fraction (``configs``).

Rooflines use MI355X published peaks: HBM 8 TB/s; dense MFMA bf16 2.5 PF/s,
fp4 10.1 PF/s.  Kernel durations come from HIP events on the stream the
kernels run on (torch's current stream).  ``traffic`` (measured HBM bytes per
launch) is read from the committed rocprof PMC summary when one exists.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP4_PEAK_TFLOPS = 10100.0
FP8_PEAK_TFLOPS = 5000.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "quantize GB/s + MXFP4 expert GEMM TFLOPS, as % of MI355X roofline (1 GPU)"


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--quick", action="store_true", help="headline only (skip the other configs)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", default="", help="comma list of sections to run (profiling)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run only a plain device copy of 1 GiB (PMC byte calibration)")
    return p.parse_args()


def _time_loop(torch, fn, steps: int, warmup: int, warm_s: float = 0.0) -> float:
    """Average seconds per call with HIP events on the current stream, after
    ``warmup`` calls and at least ``warm_s`` seconds of them (the clocks of a
    long MFMA-bound kernel settle over the first ~100 ms of sustained load)."""
    t0 = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - t0 < warm_s:
        fn()
        done += 1
        if warm_s and done % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / steps


def _bound(N, name: str, *args):
    """A C entry point with its arguments converted once: for kernels of a few
    microseconds, so the timed loop measures the GPU and not the per-call
    Python argument conversion."""
    import ctypes

    fn = getattr(N.library(), name)
    conv = tuple(ctypes.c_void_p(a) if a is None else a for a in args)

    def run():
        rc = fn(*conv)
        if rc != 0:
            raise RuntimeError(f"{name} failed ({rc}): {N.library().kq_last_error().decode()}")

    return run


def _traffic(name: str):
    path = ROOT / "profiles" / f"{name}_traffic.json"
    if path.exists():
        try:
            return json.loads(path.read_text()).get("bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


def _roofline(bound: str, achieved: float, traffic_name: str | None = None):
    peak = HBM_PEAK_GBS if bound == "hbm" else BF16_PEAK_TFLOPS
    return {
        "bound": bound,
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "traffic": _traffic(traffic_name) if traffic_name else None,
    }


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        return 2
    import torch

    from kquant_amd import _native as N
    from kquant_amd import candidate_hessian, linear, moe, mxfp8, workloads
    from kquant_amd import mxfp4 as kq_mxfp4

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    N.library()
    only = set(filter(None, args.only.split(",")))

    def want(section: str) -> bool:
        return not only or section in only

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 1 << 30, "launches": 5}))
        return 0

    stream = N.stream(dev)
    result = {}

    # ---------------------------------------------------------- headline --
    w2 = workloads.cfg2_weight().to(dev)
    rows, cols = w2.shape
    q8 = torch.empty(rows, cols, dtype=torch.uint8, device=dev)
    s8 = torch.empty(rows, cols // 32, dtype=torch.uint8, device=dev)
    quant_bytes = rows * cols * 2 + rows * cols + rows * cols // 32

    quantize_step = _bound(N, "kq_mx_quantize", N.FMT_MXFP8_E4M3, N.DT_BF16, N.ptr(w2), cols, rows, cols,
                           N.ptr(q8), N.ptr(s8), 0, stream)

    t_quant = _time_loop(torch, quantize_step, args.steps, args.warmup) if want("quantize") else float("nan")
    quant_gbs = quant_bytes / t_quant / 1e9
    if want("quantize"):
        # what a plain device copy of the same weight reaches on this box (read + write)
        copy_dst = torch.empty_like(w2)
        t_copy = _time_loop(torch, lambda: copy_dst.copy_(w2), args.steps, args.warmup)
        copy_gbs = 2 * w2.numel() * w2.element_size() / t_copy / 1e9
        result["hbm_copy_reference"] = {
            "what": "torch device copy of the cfg2 bf16 weight (176 MB read + 176 MB written)",
            "gbs": round(copy_gbs, 1),
            "quantize_over_copy": round(quant_gbs / copy_gbs, 3),
        }
        del copy_dst

    # ---------------------------------------------- config 2 GEMM (A16) --
    if not args.quick and want("linear"):
        x2 = workloads.cfg2_activations().to(dev)
        out2 = torch.empty(x2.shape[0], rows, dtype=torch.bfloat16, device=dev)

        def gemm_step():
            N.call("kq_mx_linear", N.FMT_MXFP8_E4M3, N.ptr(x2), cols, N.ptr(q8), N.ptr(s8),
                   x2.shape[0], rows, cols, N.DT_BF16, N.ptr(out2), rows, stream)

        quantize_step()
        t_gemm = _time_loop(torch, gemm_step, max(5, args.steps // 5), 3, 0.3)
        flops = 2.0 * x2.shape[0] * rows * cols
        result["cfg2_mxfp8_linear"] = {
            "workload": "X[4096x7168] bf16 @ dequant(MXFP8 W[12288x7168])^T -> bf16, fp32 accumulate",
            "tflops": round(flops / t_gemm / 1e12, 1),
            "us": round(t_gemm * 1e6, 1),
            "roofline": _roofline("mfma", flops / t_gemm / 1e12, "mx_linear_cfg2"),
        }
        del x2, out2

    # ------------------------------------------ config 3 MoE prefill GEMM --
    moe_result = None
    if not args.quick and want("moe_prefill"):
        ids, rw = workloads.zipf_routing(8192)
        active = torch.unique(ids).tolist()
        raw = workloads.quantized_experts(active, device=dev)
        weights = moe.prepare_expert_weights(*raw)
        x4t_scales = moe.prepare_expert_weights(*raw, scale_format="x4t")
        del raw
        x3 = (torch.randn(8192, workloads.HIDDEN, generator=torch.Generator().manual_seed(6))
              .to(torch.bfloat16).to(dev))
        ids_d, rw_d = ids.to(dev), rw.to(dev)

        def moe_step():
            moe.grouped_expert_forward(x3, ids_d, rw_d, weights)

        t_moe = _time_loop(torch, moe_step, max(3, args.steps // 10), 2, 0.3)
        flops = workloads.moe_flops(ids.numel())
        tflops = flops / t_moe / 1e12
        wbytes = len(active) * workloads.bytes_per_expert()
        moe_result = {
            "workload": "cfg3: 8192 tok, top-8 Zipf(1.1) over 384 experts, H=7168 I=2048, "
                        "MXFP4 W4A16 (bf16 MFMA), SiTU, fp32 out",
            "tflops": round(tflops, 1),
            "ms": round(t_moe * 1e3, 3),
            "active_experts": len(active),
            "weight_bytes": wbytes,
            "roofline": _roofline("mfma", tflops, "moe_prefill_cfg3"),
            "frac_of_fp4_dense_peak": round(tflops / FP4_PEAK_TFLOPS, 4),
        }

        # the same forward with X4T-coded expert scales (grouped-GEMM experts'
        # scales expanded per call, the GEMV experts' decoded in the GEMV)
        def moe_x4t_step():
            moe.grouped_expert_forward(x3, ids_d, rw_d, x4t_scales)

        t_x4t = _time_loop(torch, moe_x4t_step, max(3, args.steps // 10), 2, 0.3)
        moe_result["x4t_scales_ms"] = round(t_x4t * 1e3, 3)
        moe_result["x4t_added_us"] = round((t_x4t - t_moe) * 1e6, 1)
        del x4t_scales
        # Activation-quantized modes (W4A8 / W4A4, no kquant counterpart): the
        # same forward with tokens and intermediates MX-quantized, every GEMM on
        # the block-scaled fp8/fp4 MFMA; priced against that MFMA's peak
        # (E4M3 x E2M1 runs at the fp8 rate, E2M1 x E2M1 at the fp4 rate).
        for fmt, peak in (("mxfp8", FP8_PEAK_TFLOPS), ("mxfp4", FP4_PEAK_TFLOPS)):
            def mx_step(fmt=fmt):
                moe.grouped_expert_forward(x3, ids_d, rw_d, weights, activation_format=fmt)

            t_mx = _time_loop(torch, mx_step, max(3, args.steps // 10), 2, 0.3)
            tf = flops / t_mx / 1e12
            result[f"cfg3_moe_prefill_{'w4a8' if fmt == 'mxfp8' else 'w4a4'}"] = {
                "workload": f"cfg3 shapes, activations {fmt.upper()}-quantized per row, block-scaled MFMA",
                "tflops": round(tf, 1),
                "ms": round(t_mx * 1e3, 3),
                "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": peak, "unit": "TFLOP/s",
                             "frac": round(tf / peak, 4), "traffic": None},
            }
        del weights, x3

    # -------------------------------------------------- config 5 decode --
    if not args.quick and want("moe_decode"):
        dec = {}
        for tokens in (1, 4, 16):
            ids, rw = workloads.random_routing(tokens, seed=tokens)
            active = torch.unique(ids).tolist()
            raw = workloads.quantized_experts(active, device=dev)
            weights = moe.prepare_expert_weights(*raw)
            # the same experts with X4T-coded scales, expanded per call
            weights_x4t = moe.prepare_expert_weights(*raw, scale_format="x4t")
            del raw
            x5 = torch.randn(tokens, workloads.HIDDEN, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
            ids_d, rw_d = ids.to(dev), rw.to(dev)

            def dec_step():
                moe.grouped_expert_forward(x5, ids_d, rw_d, weights)

            def dec_x4t_step():
                moe.grouped_expert_forward(x5, ids_d, rw_d, weights_x4t)

            t = _time_loop(torch, dec_step, max(10, args.steps), 5)
            t_x = _time_loop(torch, dec_x4t_step, max(10, args.steps), 5)
            nbytes = len(active) * workloads.bytes_per_expert() + tokens * workloads.HIDDEN * 2
            dec[f"batch{tokens}"] = {
                "us": round(t * 1e6, 1),
                "distinct_experts": len(active),
                "gbs": round(nbytes / t / 1e9, 1),
                "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                "x4t_scales_us": round(t_x * 1e6, 1),
                "x4t_added_us": round((t_x - t) * 1e6, 1),
            }
            del weights, weights_x4t
        result["cfg5_moe_decode"] = dec

    # ------------------------------------------------- config 1 codec --
    if not args.quick and want("cfg1"):
        w1 = workloads.cfg1_weight().to(dev)
        q4 = torch.empty(7168, 1024, dtype=torch.uint8, device=dev)
        s4 = torch.empty(7168, 64, dtype=torch.uint8, device=dev)
        d4 = torch.empty(7168, 2048, dtype=torch.bfloat16, device=dev)
        b1 = 7168 * 2048 * 2 + 7168 * 1024 + 7168 * 64

        q_step = _bound(N, "kq_mx_quantize", N.FMT_MXFP4_E2M1, N.DT_BF16, N.ptr(w1), 2048, 7168, 2048,
                        N.ptr(q4), N.ptr(s4), 0, stream)
        d_step = _bound(N, "kq_mx_dequant", N.FMT_MXFP4_E2M1, N.ptr(q4), N.ptr(s4), 7168, 2048,
                        N.DT_BF16, N.ptr(d4), 0, stream)

        tq = _time_loop(torch, q_step, args.steps, args.warmup)
        td = _time_loop(torch, d_step, args.steps, args.warmup)
        result["cfg1_mxfp4_codec"] = {
            "quantize_gbs": round(b1 / tq / 1e9, 1), "quantize_us": round(tq * 1e6, 2),
            "dequant_gbs": round(b1 / td / 1e9, 1), "dequant_us": round(td * 1e6, 2),
            "hbm_frac_quantize": round(b1 / tq / 1e9 / HBM_PEAK_GBS, 4),
            "note": "37 MB working set stays within the 256 MB last-level cache across back-to-back launches",
        }

    # ---------------------------------------------- config 4 Hessian --
    if not args.quick and want("hessian"):
        g = torch.Generator(device=dev).manual_seed(0)
        x4 = (torch.randn(65536, 7168, generator=g, device=dev)
              / torch.sqrt(sum(torch.randn(65536, 7168, generator=g, device=dev).square() for _ in range(4)) / 4)
              ).to(torch.bfloat16)
        acc = torch.empty(7168, 7168, dtype=torch.float32, device=dev)

        def h_step():
            N.call("kq_syrk_accumulate", N.DT_BF16, N.ptr(x4), 7168, 65536, 7168, N.ptr(None),
                   N.ptr(acc), 7168, N.SYRK_OVERWRITE, stream)

        th = _time_loop(torch, h_step, 3, 1)
        flops = workloads.syrk_flops(65536, 7168)
        result["cfg4_hessian_k7168"] = {
            "tflops": round(flops / th / 1e12, 1),
            "ms": round(th * 1e3, 3),
            "roofline": _roofline("mfma", flops / th / 1e12, "syrk_cfg4"),
        }
        del x4, acc

    # --------------------------- config 4 (ii) per-expert Hessians, K=2048 --
    if not args.quick and want("hessian_experts"):
        ids, rw = workloads.zipf_routing(65536)
        experts = workloads.EXPERTS
        counts = torch.bincount(ids[ids >= 0].flatten().long(), minlength=experts)
        offsets = torch.zeros(experts + 1, dtype=torch.int64)
        offsets[1:] = torch.cumsum(counts, 0)
        pairs = int(offsets[-1])
        k2 = workloads.INTER
        g = torch.Generator(device=dev).manual_seed(1)
        rows = torch.empty(pairs, k2, dtype=torch.bfloat16, device=dev)
        for c0 in range(0, pairs, 65536):  # Student-t(4) rows, generated in slabs
            n = min(65536, pairs - c0)
            z = torch.randn(n, k2, generator=g, device=dev)
            chi = sum(torch.randn(n, k2, generator=g, device=dev).square() for _ in range(4))
            rows[c0:c0 + n] = (z / torch.sqrt(chi / 4)).to(torch.bfloat16)
        gates = torch.rand(pairs, generator=g, device=dev)
        offsets_d = offsets.to(dev)
        hacc = torch.empty(experts, k2, k2, dtype=torch.float32, device=dev)

        def he_step():
            N.call("kq_syrk_grouped", N.DT_BF16, N.ptr(rows), k2, N.ptr(offsets_d), experts, None,
                   N.ptr(gates), k2, N.ptr(hacc), N.SYRK_SQUARE_WEIGHTS, stream)

        the = _time_loop(torch, he_step, 3, 1)
        flops = float((counts.double() * k2 * (k2 + 1)).sum())
        hbytes = pairs * k2 * 2 + pairs * 4 + experts * k2 * k2 * 4
        result["cfg4_hessian_experts_k2048"] = {
            "workload": "cfg4 (ii): gate^2-weighted X^T X of each expert's routed rows, 65536 tokens "
                        "top-8 Zipf(1.1) over 384 experts (524288 rows of 2048 bf16), one grouped launch",
            "ms": round(the * 1e3, 3),
            "tflops": round(flops / the / 1e12, 1),
            "gbs": round(hbytes / the / 1e9, 1),
            "roofline": _roofline("hbm", hbytes / the / 1e9),
            "active_experts": int((counts > 0).sum()),
        }
        del rows, hacc

    # ------------------------------- encoder H finalize (rotation, block LDL) --
    if not args.quick and want("h_finalize"):
        def spd(batch: int, n: int, seed: int) -> torch.Tensor:
            gh = torch.Generator(device=dev).manual_seed(seed)
            out = torch.empty(batch, n, n, dtype=torch.float32, device=dev)
            for b in range(batch):
                xs = torch.randn(2 * n, n, generator=gh, device=dev)
                h = xs.T @ xs / (2 * n)
                out[b] = h + 0.025 * torch.diagonal(h).mean() * torch.eye(n, device=dev)
            return out

        def chol_ws(n: int, batch: int) -> torch.Tensor:
            return torch.empty(int(N.library().kq_cholesky_workspace_size(n, batch)), dtype=torch.uint8,
                               device=dev)

        fin = {}
        for label, batch, n in (("h13_k7168", 1, 7168), ("h2_experts48_k2048", 48, 2048)):
            h = spd(batch, n, 3)
            lower = torch.empty_like(h)
            info = torch.empty(batch, dtype=torch.int32, device=dev)
            wsc = chol_ws(n, batch)
            wsl = torch.empty(int(N.library().kq_block_ldl_workspace_size(n, 16, batch)), dtype=torch.uint8,
                              device=dev)
            su = torch.ones(n, dtype=torch.float32, device=dev)
            mean = torch.empty(1, dtype=torch.float32, device=dev)

            def rot_step():
                for b in range(batch):
                    N.call("kq_h_regularize", N.ptr(h[b]), n, n, 1.0, 1e-6, None, N.ptr(mean), stream)
                N.call("kq_blockwise_hadamard", N.ptr(h), n, n, n, batch, n * n, 3, N.ptr(su), N.ptr(su), stream)

            def chol_step():
                N.call("kq_cholesky", N.ptr(h), n, n * n, N.ptr(lower), n, n * n, n, batch, N.ptr(info),
                       N.ptr(wsc), wsc.numel(), stream)

            def ldl_step():
                N.call("kq_block_ldl", N.ptr(lower), n, n * n, n, 16, batch, N.LDL_ZERO_DIAGONAL, N.ptr(wsl),
                       wsl.numel(), stream)

            t_rot = _time_loop(torch, rot_step, 3, 1)
            t_chol = _time_loop(torch, chol_step, 3, 1)
            ldl_step()
            t_ldl = _time_loop(torch, ldl_step, 3, 1)
            t_torch = _time_loop(torch, lambda: torch.linalg.cholesky(h), 3, 1)
            flops = batch * n ** 3 / 3.0
            fin[label] = {
                "matrices": batch, "n": n,
                "regularize_rotate_ms": round(t_rot * 1e3, 3),
                "cholesky_ms": round(t_chol * 1e3, 3),
                "cholesky_tflops": round(flops / t_chol / 1e12, 2),
                "cholesky_frac_of_fp32_mfma_peak": round(flops / t_chol / 1e12 / FP32_PEAK_TFLOPS, 4),
                "block_ldl_ms": round(t_ldl * 1e3, 3),
                "torch_linalg_cholesky_ms": round(t_torch * 1e3, 3),
            }
            del h, lower
        result["h_finalize"] = fin

    # ------------------------------ QSRT trellis: SQG encoder and weight decode --
    if not args.quick and want("qsrt"):
        from kquant_amd import qsrt as kq_qsrt
        from kquant_amd import sqg_quantizer
        from kquant_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

        qres = {}
        gq = torch.Generator(device=dev).manual_seed(7)
        n_enc = 2048
        xt = torch.randn(n_enc, 256, generator=gq, device=dev)
        for bits in (2, 3, 4):
            lut = sqg_xor_cheb_t12_bytes(bits, device=dev)

            def enc_step(lut=lut, bits=bits):
                sqg_quantizer.quantize_tiles_sqg(xt, lut, bits, 128)

            t_enc = _time_loop(torch, enc_step, 2, 1)
            qres[f"sqg_encode_k{bits}"] = {
                "tiles": n_enc,
                "ms": round(t_enc * 1e3, 2),
                "tiles_per_s": round(n_enc / t_enc, 1),
                # 512 steps (256-step primer + closing pass) x 65536 edges per tile
                "edge_evals_per_s": round(n_enc * 512 * 65536 / t_enc / 1e12, 3),
                "unit": "edge_evals T/s",
            }
        # decode of one Kimi-K3 w1 matrix: EXL [K=3584, N=3072], rate axis n, P24 x 2 + P33 x 10
        k_tiles, n_tiles = 224, 192
        record_bits = (2, 4) * 2 + (3,) * 20
        words = sum(8 * k_tiles * 16 * b for b in record_bits)
        payload = torch.randint(-32768, 32768, (words,), dtype=torch.int16, generator=gq, device=dev)
        suh = torch.ones(k_tiles * 16, device=dev)
        svh = torch.ones(n_tiles * 16, device=dev)

        def dec_qsrt():
            kq_qsrt.decode_qsrt_payload(payload, k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n",
                                        record_bits=record_bits, suh=suh, svh=svh, out_dtype=torch.bfloat16,
                                        transposed=True)

        t_dq = _time_loop(torch, dec_qsrt, 20, 3)
        dbytes = words * 2 + k_tiles * n_tiles * 256 * 2
        qres["qsrt_decode_w1_k3"] = {
            "workload": "QSRT w1 [3072 x 3584] (R2: 2 x P24 + 10 x P33) -> bf16 [N, K], rotation included",
            "us": round(t_dq * 1e6, 1),
            "gbs": round(dbytes / t_dq / 1e9, 1),
            "hbm_frac": round(dbytes / t_dq / 1e9 / HBM_PEAK_GBS, 4),
        }
        # the fused linear on the same matrix (x @ W without materializing W)
        # and on the TP12-local expert shapes of the same checkpoint
        lin_cases = {
            "k3_w1": (k_tiles, n_tiles, "n", record_bits, payload, suh, svh),
        }
        for name, kt_, nt_, axis, bits_ in (("tp12_w13", 224, 32, "n", (3,) * 4), ("tp12_w2", 16, 224, "k", (3, 3))):
            w_ = sum(8 * (kt_ if axis == "n" else nt_) * 16 * b for b in bits_)
            lin_cases[name] = (kt_, nt_, axis, bits_,
                               torch.randint(-32768, 32768, (w_,), dtype=torch.int16, generator=gq, device=dev),
                               torch.ones(kt_ * 16, device=dev), torch.ones(nt_ * 16, device=dev))
        lin = {}
        reps = 20
        for name, (kt_, nt_, axis, bits_, p_, su_, sv_) in lin_cases.items():
            row = {}
            for m in (1, 4, 16):
                xq = torch.randn(m, kt_ * 16, generator=gq, device=dev).to(torch.bfloat16)
                outq = torch.empty(m, nt_ * 16, dtype=torch.bfloat16, device=dev)
                run = kq_qsrt.qsrt_linear_launcher(xq, p_, outq, k_tiles=kt_, n_tiles=nt_, rate_axis=axis,
                                                   record_bits=bits_, suh=su_, svh=sv_)
                run()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    for _ in range(reps):
                        run()
                row[f"m{m}_us"] = round(_time_loop(torch, graph.replay, 10, 3) / reps * 1e6, 2)
            row["weight_bytes"] = int(p_.numel() * 2)
            lin[name] = row
        # routed experts at the Kimi-K3 TP12-local geometry (H = 3584, 256
        # intermediate channels per rank, top-16), QSRT P33-like rates (K3)
        h_, i_, n_exp, topk_ = 3584, 256, 64, 16

        def rand_mat(k, n, axis, bits_each):
            records = (k if axis == "k" else n) // 128
            per = 8 * ((n if axis == "k" else k) // 16)
            w_ = per * 16 * bits_each * records
            return (torch.randint(-32768, 32768, (w_,), dtype=torch.int16, generator=gq, device=dev),
                    (bits_each,) * records, torch.randn(k, generator=gq, device=dev).sign(),
                    torch.rand(n, generator=gq, device=dev) + 0.5)

        mats_ = [[rand_mat(h_, i_, "n", 3), rand_mat(h_, i_, "n", 3), rand_mat(i_, h_, "k", 3)] for _ in range(n_exp)]
        qexp = kq_qsrt.QSRTExperts([m[0] for m in mats_], [m[1] for m in mats_], [m[2] for m in mats_],
                                   hidden=h_, inter=i_)
        moe_q = {}
        for toks in (1, 4):
            xq = torch.randn(toks, h_, generator=gq, device=dev).to(torch.bfloat16)
            ids_ = torch.stack([torch.randperm(n_exp, generator=torch.Generator().manual_seed(t))[:topk_]
                                for t in range(toks)]).to(device=dev, dtype=torch.int32)
            wts_ = torch.rand(toks, topk_, generator=gq, device=dev)
            kq_qsrt.qsrt_expert_forward(xq, ids_, wts_, qexp)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(reps):
                    kq_qsrt.qsrt_expert_forward(xq, ids_, wts_, qexp)
            moe_q[f"tokens{toks}_us"] = round(_time_loop(torch, graph.replay, 10, 3) / reps * 1e6, 2)
        qres["qsrt_moe_decode_tp12"] = {
            "workload": "routed expert forward, H=3584, I=256 per rank, top-16, QSRT K3 w1/w3/w2, bf16 in/out, "
                        "fp32 math; time per forward from a HIP graph of 20",
            **moe_q,
            "reference_split_k_w4a16_qsrt_us": {"P33": 56.90, "P24": 65.09},
        }
        qres["qsrt_linear"] = {
            "workload": "x[m, K] bf16 @ QSRT W (rotated, fp32 math) -> bf16; time per call from a HIP "
                        "graph of 20 back-to-back calls",
            **lin,
        }
        result["qsrt"] = qres

    # ------------------------------------- scale-plane codecs and SQG tables --
    if not args.quick and want("scale_planes"):
        from kquant_amd import sqg_e4m3
        w1 = workloads.cfg1_weight().to(dev)
        _, plane = kq_mxfp4.mxfp4_quantize(w1)          # [7168, 64] E8M0 plane
        prows, pcols = plane.shape
        tiles = prows // 16
        fixed = torch.empty(tiles * 16 * (1 + pcols // 8), dtype=torch.uint8, device=dev)
        toff = torch.empty(tiles + 1, dtype=torch.int64, device=dev)
        N.call("kq_x4t_analyze", N.ptr(plane), 1, prows, pcols, N.ptr(fixed), N.ptr(toff), stream)
        n_exc = int(toff[-1].item())
        exc = torch.empty(max(n_exc, 1), dtype=torch.uint32, device=dev)
        out_plane = torch.empty_like(plane)

        def x4t_pack():
            N.call("kq_x4t_analyze", N.ptr(plane), 1, prows, pcols, N.ptr(fixed), N.ptr(toff), stream)
            N.call("kq_x4t_emit_exceptions", N.ptr(plane), 1, prows, pcols, N.ptr(fixed), N.ptr(toff),
                   N.ptr(exc), stream)

        def x4t_decode():
            N.call("kq_x4t_decode", N.ptr(fixed), N.ptr(exc), n_exc, None, 1, prows, pcols,
                   N.ptr(out_plane), None, stream)

        t_xp = _time_loop(torch, x4t_pack, 50, 5)
        t_xd = _time_loop(torch, x4t_decode, 50, 5)
        meta = torch.empty(prows, dtype=torch.int32, device=dev)
        koff = torch.empty(prows // 16 + 1, dtype=torch.int64, device=dev)
        N.call("kq_kqsc_measure", 2, N.ptr(plane), prows, pcols, 16, N.ptr(meta), N.ptr(koff), stream)
        payload = torch.empty(16 + 4 * (prows // 16 + 1) + int(koff[-1].item()), dtype=torch.uint8,
                              device=dev)
        kstatus = torch.empty(1, dtype=torch.int64, device=dev)

        def kqsc_pack():
            N.call("kq_kqsc_measure", 2, N.ptr(plane), prows, pcols, 16, N.ptr(meta), N.ptr(koff), stream)
            N.call("kq_kqsc_emit", 2, N.ptr(plane), prows, pcols, 16, N.ptr(meta), N.ptr(koff),
                   N.ptr(payload), stream)

        def kqsc_decode():
            N.call("kq_kqsc_decode", 2, N.ptr(payload), payload.numel(), prows, pcols, 16,
                   N.ptr(out_plane), N.ptr(kstatus), stream)

        t_kp = _time_loop(torch, kqsc_pack, 50, 5)
        t_kd = _time_loop(torch, kqsc_decode, 50, 5)
        t0 = time.perf_counter()
        sqg_e4m3._normal_law.cache_clear()
        sqg_e4m3._t12.cache_clear()
        sqg_e4m3._xor_t12_labels.cache_clear()
        sqg_e4m3._rank.cache_clear()
        labels = sqg_e4m3.sqg_xor_cheb_t12_bytes(3, device=dev)
        torch.cuda.synchronize()
        t_sqg = time.perf_counter() - t0
        result["scale_planes_cfg1"] = {
            "workload": "E8M0 plane [7168x64] of the cfg1 MXFP4 weight",
            "x4t_exceptions": n_exc,
            "x4t_pack_us": round(t_xp * 1e6, 2),
            "x4t_predecode_us": round(t_xd * 1e6, 2),
            "kqsc_v2_bytes": int(payload.numel()),
            "kqsc_v2_pack_us": round(t_kp * 1e6, 2),
            "kqsc_v2_decode_us": round(t_kd * 1e6, 2),
            "sqg_k3_t12_labels_build_ms": round(t_sqg * 1e3, 3),
            "sqg_labels": int(labels.numel()),
        }

    # ------------------------------------------------- CPU baseline --
    cpu = None
    if not args.no_cpu_baseline and want("cpu"):
        from oracle import torch_ref

        torch.set_num_threads(min(os.cpu_count() or 1, 16))
        w_cpu = workloads.cfg2_weight()
        sample_rows = 3072  # a quarter of the matrix: ~5-20 s of CPU work over 5 runs
        sample = w_cpu[:sample_rows].contiguous()
        torch_ref.mxfp8_quantize_cpu(sample)
        times = []
        for _ in range(5):
            t0 = time.perf_counter()
            torch_ref.mxfp8_quantize_cpu(sample)
            times.append(time.perf_counter() - t0)
        tmed = statistics.median(times)
        sbytes = sample_rows * cols * 2 + sample_rows * cols + sample_rows * cols // 32
        cpu = {
            "value": round(sbytes / tmed / 1e9, 3),
            "unit": "GB/s",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"kquant/mxfp8.py:34-50 formula on torch CPU ops, rows 0..{sample_rows} of the "
                      f"cfg2 weight (bf16 [{sample_rows}x{cols}]), median of 5 runs",
            "cpu": platform.processor() or platform.machine(),
        }

    line = {
        "metric": METRIC,
        "value": round(quant_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_quant * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16->e4m3",
        "data": "synthetic (seeded N(0,0.015) bf16 weight, BASELINE config 2)",
        "config": {
            "workload": "cfg2: MXFP8 E4M3 quantize of W[12288x7168] bf16 (32-elem blocks, E8M0 scale)",
            "bytes_per_step": quant_bytes,
            "parallelism": "1 GPU",
        },
        "roofline": _roofline("hbm", quant_gbs, "mx_quantize_cfg2"),
        "cpu_baseline": cpu,
        "moe_prefill": moe_result,
        "configs": result,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
