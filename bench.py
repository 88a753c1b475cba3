"""Benchmark of the MI355X quantized-inference hot path on one GPU.

Headline: the fused fp16 attention configuration (B=1, H=24, S=4096, D=128, no mask, scale 1/sqrt(128)); one step
is one call of hip_attention.attention (a single kernel launch) with Q/K/V resident in HBM. `value` is achieved
TFLOP/s over the timed steps (4 B H S^2 D = 206.16 GFLOP per step). The other configurations of the metric -- the
W8A8 linear (int8 GEMM TOPS), int8-QK attention, W4A8 linear, the DiT MLP tail and the decode GEMV / attention
(HBM GB/s) -- are measured in the same run and reported under "components".

Kernel durations come from HIP events recorded around every launch on torch's current stream (the stream every
entry point of the library launches on). HBM-bound kernels rotate over enough input copies (> 512 MB) that
the 256 MB Infinity Cache cannot serve them. The CPU baseline is the reference's own fallback for attention
(attention_bmm: chunked baddbmm -> softmax -> bmm, attention.py:15-43) run by torch on the host cores over a
bounded sample of heads.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-components] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int8 GEMM TOPS (% MFMA peak), attn fp16 TFLOPS, GEMV HBM GB/s, 1 MI355X"
# MI355X peaks (256 CUs at 2.4 GHz; dense matrix rates): fp16 4096 and int8 8192 ops/CU/clock.
PEAK_F16_TFLOPS = 2516.6
PEAK_I8_TOPS = 5033.2
PEAK_HBM_GBS = 8000.0
ROTATE_BYTES = 640 * 2 ** 20  # > 2x the Infinity Cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """Per-launch HIP events on the current stream."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def __call__(self, fn):
        s = self.torch.cuda.Event(enable_timing=True)
        e = self.torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn()
        e.record()
        self.pairs.append((s, e))
        return out

    def mean_ms(self):
        self.torch.cuda.synchronize()
        return sum(s.elapsed_time(e) for s, e in self.pairs) / len(self.pairs)


def timed(torch, fn, steps, warmup, copies=1):
    """Runs fn(i) warmup + steps times; returns (wall ms per step, mean kernel ms from per-launch events)."""
    for i in range(warmup):
        fn(i % copies)
    torch.cuda.synchronize()
    timer = Timer(torch)
    t0 = time.perf_counter()
    for i in range(steps):
        timer(lambda: fn(i % copies))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, timer.mean_ms()


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic}


def gen(torch, seed):
    return torch.Generator().manual_seed(seed)


def attention_inputs(torch, dev):
    B, H, S, D = 1, 24, 4096, 128
    q = torch.randn(B, H, S, D, generator=gen(torch, 4)).half()
    k = torch.randn(B, H, S, D, generator=gen(torch, 5)).half()
    v = torch.randn(B, H, S, D, generator=gen(torch, 6)).half()
    return q, k, v


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


def cpu_baseline(torch, q, k, v):
    """The reference's attention fallback on the host cores: fp32 over 4 of the 24 heads at full length, fp16 over
    one head with 1024 of its query rows (torch's CPU fp16 matmul is far slower); the faster rate is reported."""
    import oracle
    threads = torch.get_num_threads()
    S, D = q.shape[2], q.shape[3]
    best = None
    for dtype, heads, rows in ((torch.float32, 4, S), (torch.float16, 1, 1024)):
        qs = q[:, :heads, :rows].to(dtype).contiguous()
        ks, vs = (t[:, :heads].to(dtype).contiguous() for t in (k, v))
        oracle.attention_bmm_cpu(qs[:, :1, :128], ks[:, :1], vs[:, :1], 128 ** -0.5)  # warm-up
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.attention_bmm_cpu(qs, ks, vs, 128 ** -0.5)
            times.append(time.perf_counter() - t0)
        rate = 4.0 * heads * rows * S * D / min(times) / 1e12
        log(f"cpu attention_bmm {dtype}: {rate:.4f} TFLOP/s ({heads} heads x {rows} rows, best of 3: {min(times):.2f} s)")
        if best is None or rate > best[0]:
            best = (rate, str(dtype).replace("torch.", ""), heads, rows)
    return {"value": round(best[0], 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"attention_bmm (chunked baddbmm/softmax/bmm in {best[1]}) over {best[2]} of 24 heads x {best[3]} query rows, "
                      f"S=4096, D=128; best of 3 after a warm-up; {os.cpu_count()} logical CPUs visible"}


def components(torch, dev, steps, warmup, traffic):
    import numpy as np  # noqa: F401
    from comfyui_rdna2_attention_amd import _lib, hip_attention, int8_gemm, int8_gemv, rms_norm
    out = {}
    k = int8_gemm.get_kernels()
    p = _lib.ptr

    # W8A8 linear: X fp16 [4096, 3072] with 8 outlier channels x30, 128-block Hadamard, W int8 [3072, 3072].
    M, K, N = 4096, 3072, 3072
    g = gen(torch, 1)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:8]] *= 30
    x = x.half().to(dev)
    w = torch.randint(-127, 128, (N, K), generator=gen(torch, 2), dtype=torch.int8).to(dev)
    ws = (torch.rand(N, generator=gen(torch, 3)) * 2e-3 + 1e-3).float().to(dev)
    act = int8_gemm.quantize(k.rot_quant_pack_a, x, K, group=128)
    c = torch.empty(M, N, dtype=torch.float16, device=dev)
    gemm = lambda i: _lib.check(k.gemm(p(act[0]), p(w), p(act[1]), p(ws), None, p(c), M, N, K, None, None, 1, _lib.stream()))  # noqa: E731
    wall, kms = timed(torch, gemm, steps, warmup)
    ops = 2.0 * M * N * K
    out["w8a8_gemm"] = {"value": round(ops / kms / 1e9, 1), "unit": "TOP/s", "kernel_ms": round(kms, 4),
                        "roofline": roofline("mfma", ops / kms / 1e9, PEAK_I8_TOPS, "TFLOP/s", traffic.get("w8a8_gemm"))}
    ncopy = max(1, ROTATE_BYTES // (M * K * 3))
    xs = [x] + [x.clone() for _ in range(ncopy - 1)]
    aq, sc = int8_gemm.quantized(M, K, dev)
    quant = lambda i: _lib.check(k.rot_quant_pack_a(p(xs[i]), K, p(aq), p(sc), M, K, 128, _lib.stream()))  # noqa: E731
    wall, qms = timed(torch, quant, steps, warmup, len(xs))
    qbytes = M * K * 2 + M * K + M * 4
    out["w8a8_rot_quant"] = {"value": round(qbytes / qms / 1e6, 1), "unit": "GB/s", "kernel_ms": round(qms, 4),
                             "roofline": roofline("hbm", qbytes / qms / 1e6, PEAK_HBM_GBS, "GB/s", traffic.get("w8a8_rot_quant"))}
    lin = lambda i: int8_gemm.linear(xs[i], w, ws, None, rotate=True, group=128)  # noqa: E731
    wall, _ = timed(torch, lin, steps, warmup, len(xs))
    out["w8a8_linear"] = {"value": round(ops / wall / 1e9, 1), "unit": "TOP/s", "ms": round(wall, 4), "note": "rotate-quant + GEMM, wall clock"}
    del xs, act, c
    log(f"w8a8: gemm {out['w8a8_gemm']['value']} TOP/s, rot-quant {out['w8a8_rot_quant']['value']} GB/s, linear {out['w8a8_linear']['value']} TOP/s")

    # int8-QK attention on the attention configuration.
    q, kk, v = (t.to(dev) for t in attention_inputs(torch, dev))
    o = torch.empty_like(q)
    flop = 4.0 * 24 * 4096 ** 2 * 128
    wall, _ = timed(torch, lambda i: hip_attention.attention(q, kk, v, o, 128 ** -0.5, True), steps, warmup)
    out["attention_i8qk"] = {"value": round(flop / wall / 1e9, 1), "unit": "TFLOP/s", "ms": round(wall, 4),
                             "roofline": roofline("mfma", flop / wall / 1e9, PEAK_F16_TFLOPS, "TFLOP/s"),
                             "note": "K quantization pass + attention, wall clock; fp16-peak roofline"}
    del q, kk, v, o
    log(f"attention int8-QK: {out['attention_i8qk']['value']} TFLOP/s")

    # W4A8 linear: W int4 [12288, 3072], group-128 fp16 scales.
    N4 = 12288
    w4 = torch.randint(0, 256, (N4, K // 2), generator=gen(torch, 8), dtype=torch.uint8).to(dev)
    gs = (torch.rand(N4, K // 128, generator=gen(torch, 9)) * 1.5e-2 + 5e-3).half().to(dev)
    act = int8_gemm.quantize(k.rot_quant_pack_a, x, K)
    c4 = torch.empty(M, N4, dtype=torch.float16, device=dev)
    w4a8 = lambda i: _lib.check(k.gemm_w4a8(p(act[0]), p(w4), p(act[1]), p(gs), None, p(c4), M, N4, K, 128, _lib.stream()))  # noqa: E731
    wall, kms = timed(torch, w4a8, steps, warmup)
    ops4 = 2.0 * M * N4 * K
    out["w4a8_gemm"] = {"value": round(ops4 / kms / 1e9, 1), "unit": "TOP/s", "kernel_ms": round(kms, 4),
                        "roofline": roofline("mfma", ops4 / kms / 1e9, PEAK_I8_TOPS, "TFLOP/s", traffic.get("w4a8_gemm"))}
    del w4, c4, act
    log(f"w4a8 gemm: {out['w4a8_gemm']['value']} TOP/s")

    # DiT MLP tail: RMSNorm [4096, 3072], SwiGLU -> rotate -> quant [4096, 8192], down GEMM K=8192, N=3072.
    hn = torch.randn(1, M, K, generator=gen(torch, 10)).half().to(dev)
    nw = (torch.randn(K, generator=gen(torch, 11)) * 0.1).float().to(dev)
    hs = [hn] + [hn.clone() for _ in range(ROTATE_BYTES // (M * K * 4))]
    wall, nms = timed(torch, lambda i: rms_norm.rms_norm(hs[i], nw, 1e-6), steps, warmup, len(hs))
    nbytes = M * K * 4 + K * 4
    out["mlp_rms_norm"] = {"value": round(nbytes / nms / 1e6, 1), "unit": "GB/s", "kernel_ms": round(nms, 4),
                           "roofline": roofline("hbm", nbytes / nms / 1e6, PEAK_HBM_GBS, "GB/s", traffic.get("mlp_rms_norm"))}
    del hs, hn
    F = 8192
    gts = [(torch.randn(M, F, generator=gen(torch, 12 + 2 * i)).half().to(dev), torch.randn(M, F, generator=gen(torch, 13 + 2 * i)).half().to(dev))
           for i in range(max(1, ROTATE_BYTES // (M * F * 4)))]
    aq, sc = int8_gemm.quantized(M, F, dev)
    sw = lambda i: _lib.check(k.swiglu_rot_quant_pack_a(p(gts[i][0]), p(gts[i][1]), p(aq), p(sc), M, F, 256, _lib.stream()))  # noqa: E731
    wall, sms = timed(torch, sw, steps, warmup, len(gts))
    sbytes = M * F * 4 + M * F + M * 4
    out["mlp_swiglu_rot_quant"] = {"value": round(sbytes / sms / 1e6, 1), "unit": "GB/s", "kernel_ms": round(sms, 4),
                                   "roofline": roofline("hbm", sbytes / sms / 1e6, PEAK_HBM_GBS, "GB/s", traffic.get("mlp_swiglu_rot_quant"))}
    del gts
    wd = torch.randint(-127, 128, (K, F), generator=gen(torch, 14), dtype=torch.int8).to(dev)
    wds = (torch.rand(K, generator=gen(torch, 15)) * 2e-3 + 1e-3).float().to(dev)
    cd = torch.empty(M, K, dtype=torch.float16, device=dev)
    down = lambda i: _lib.check(k.gemm(p(aq), p(wd), p(sc), p(wds), None, p(cd), M, K, F, None, None, 1, _lib.stream()))  # noqa: E731
    wall, dms = timed(torch, down, steps, warmup)
    dops = 2.0 * M * K * F
    out["mlp_down_gemm"] = {"value": round(dops / dms / 1e9, 1), "unit": "TOP/s", "kernel_ms": round(dms, 4),
                            "roofline": roofline("mfma", dops / dms / 1e9, PEAK_I8_TOPS, "TFLOP/s", traffic.get("mlp_down_gemm"))}
    del wd, cd
    log(f"mlp tail: norm {out['mlp_rms_norm']['value']} GB/s, swiglu-quant {out['mlp_swiglu_rot_quant']['value']} GB/s, "
        f"down {out['mlp_down_gemm']['value']} TOP/s")

    # Decode: int8 GEMV K=4096, fp16 activations, N in {4096, 1024, 12288}; fp32 GQA decode attention.
    Kd = 4096
    xd = torch.randn(1, Kd, generator=gen(torch, 16)).half().to(dev)
    for Nd in (4096, 1024, 12288):
        copies = max(1, ROTATE_BYTES // (Nd * Kd))
        wq = torch.randint(-127, 128, (Nd, Kd), generator=gen(torch, 17), dtype=torch.int8).to(dev)
        wqs = [wq] + [wq.clone() for _ in range(copies - 1)]
        sd = (torch.rand(Nd, generator=gen(torch, 18)) * 2e-3 + 1e-3).float().to(dev)
        yd = torch.empty(1, Nd, dtype=torch.float16, device=dev)
        k_gemv = int8_gemv.get_kernels().gemv_i8
        gv = lambda i: _lib.check(k_gemv(p(xd), 1, p(wqs[i]), p(sd), None, p(yd), Nd, Kd, _lib.stream()))  # noqa: E731
        wall, gms = timed(torch, gv, max(steps, 200), warmup, len(wqs))
        gbytes = Nd * Kd + Nd * 4 + Kd * 2 + Nd * 2
        out[f"decode_gemv_n{Nd}"] = {"value": round(gbytes / gms / 1e6, 1), "unit": "GB/s", "kernel_ms": round(gms, 5),
                                     "roofline": roofline("hbm", gbytes / gms / 1e6, PEAK_HBM_GBS, "GB/s", traffic.get(f"decode_gemv_n{Nd}"))}
        del wqs, wq
        log(f"gemv N={Nd}: {out[f'decode_gemv_n{Nd}']['value']} GB/s ({gms * 1e3:.2f} us)")
    cap, H, Hkv = 2048, 32, 8
    qd = torch.randn(1, 1, H, 128, generator=gen(torch, 19)).float().to(dev)
    kvs = [(torch.randn(1, cap, Hkv, 128, generator=gen(torch, 20)).float().to(dev), torch.randn(1, cap, Hkv, 128, generator=gen(torch, 21)).float().to(dev))]
    kvs += [(a.clone(), b.clone()) for a, b in kvs * (ROTATE_BYTES // (2 * cap * Hkv * 512) - 1)]
    ln = torch.tensor([cap], dtype=torch.int32, device=dev)
    wall, _ = timed(torch, lambda i: int8_gemv.attention_decode(qd, kvs[i][0], kvs[i][1], ln), max(steps, 200), warmup, len(kvs))
    abytes = 2 * cap * Hkv * 512 + 2 * H * 512
    out["decode_attention"] = {"value": round(abytes / wall / 1e6, 1), "unit": "GB/s", "ms": round(wall, 5),
                               "roofline": roofline("hbm", abytes / wall / 1e6, PEAK_HBM_GBS, "GB/s"), "note": "decode + merge launches, wall clock"}
    log(f"decode attention: {out['decode_attention']['value']} GB/s")
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__
    __graft_entry__.load_package()
    from comfyui_rdna2_attention_amd import hip_attention

    dev = torch.device("cuda:0")
    q, k, v = attention_inputs(torch, dev)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    out = torch.empty_like(qd)
    scale = 128 ** -0.5
    flop = 4.0 * 24 * 4096 ** 2 * 128
    step = lambda i: hip_attention.attention(qd, kd, vd, out, scale)  # noqa: E731
    log(f"attention fp16 B=1 H=24 S=4096 D=128: warmup {args.warmup}, steps {args.steps}")
    wall, kms = timed(torch, step, args.steps, args.warmup)
    traffic = load_traffic()
    result = {
        "metric": METRIC,
        "value": round(flop / wall / 1e9, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "fused attention fp16, no mask: B=1, H=24, S=4096, D=128, Q/K/V ~ N(0,1), scale 1/sqrt(128)",
                   "B": 1, "H": 24, "S": 4096, "D": 128},
        "roofline": roofline("mfma", flop / kms / 1e9, PEAK_F16_TFLOPS, "TFLOP/s", traffic.get("attention_f16")),
        "kernel_ms": round(kms, 5),
    }
    log(f"attention fp16: {result['value']} TFLOP/s wall, kernel {kms:.4f} ms ({result['roofline']['frac'] * 100:.1f}% of fp16 peak)")
    del qd, kd, vd, out
    if not args.no_components:
        result["components"] = components(torch, dev, args.steps, args.warmup, traffic)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, q, k, v)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
