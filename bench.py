#!/usr/bin/env python3
"""Throughput of the fused GGUF dequantize-and-multiply path on one MI355X.

Headline workload (the JSON line's `value`): one decode token (M = 1) through all 80 layers
of a Llama-3-70B Q4_K_M model whose weights are distinct random tensors resident in HBM
(q/k/v/o/gate/up in Q4_K, down in Q6_K; 43.35 GB).  A step issues the 7 projections of
every layer (560 GEMVs) back to back on one stream through `qmm_gemm_batch`, which runs q/k/v
and gate/up (each set reads the same activations) as one launch each: 4 launches per layer.
Activations and outputs are fp16, the dtype of the reference's `matmul_q4_k` interface.
`value` is algorithmic bytes (packed weights + fp16 activations read once per GEMV + fp16
outputs written once) per second over the timed steps.

The `roofline` object covers the dominant kernel, the fused gate+up launch (two Q4_K
28672 x 8192 GEMVs on one activation vector): its 80 launches of one step are issued back to
back between two HIP events on their stream, and `achieved` is its algorithmic bytes over the
average launch duration; `traffic` is the HBM bytes per launch from the committed counter
summary (profiles/gemv_q4_k_gate_up_2x28672x8192_m1_traffic.md, made with `--pmc-workload`).
`cpu_baseline` times the in-repo NumPy restatement of the reference's CPU path (dequantize to
fp16, then fp32 matmul) on every configuration, dequantization and matmul reported apart; its
`value` is one 70B Q4_K_M layer at M = 1.  `extra` holds the other configurations (8B
Q8_0 / Q4_K_M layers, the 8B Q6_K lm_head and token-embedding gather-dequant, 70B at M = 4, the
Q4_0 4096 x 4096 case, prefill M = 512 with the vendor f16 GEMM on dense weights beside it), the
GEMV ones on rotated weight copies larger than the 256 MB MALL.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-extra] [--no-cpu-baseline] [--pmc-workload]
       [--full-layers-only]
       [--prefill-only]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "gfx1150-inference_amd")
for _p in (PKG, os.path.join(REPO, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
F16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_specs(hidden, inter, kv, main, down):
    """(name, type, N, K, input) of the 7 projections of one transformer layer.  Inputs follow a
    layer's dataflow: q/k/v read the normed hidden state, o the attention output, gate/up the
    post-attention normed state, down the SwiGLU output (so only q/k/v and gate/up can share a
    launch)."""
    return [("q", main, hidden, hidden, "h"), ("k", main, kv, hidden, "h"), ("v", main, kv, hidden, "h"),
            ("o", main, hidden, hidden, "attn"), ("gate", main, inter, hidden, "h2"), ("up", main, inter, hidden, "h2"),
            ("down", down, hidden, inter, "f")]


def weight_bytes(t, n, k):
    qk, bb = BLOCK[t]
    return n * (k // qk) * bb


class Hip:
    """hipEvent helpers from the HIP runtime already loaded by torch (same runtime as libqmm)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        rc = self.lib.hipEventCreate(ctypes.byref(e))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed ({rc})")
        return e.value

    def record(self, e, stream):
        if self.lib.hipEventRecord(e, stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        if self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, e):
        self.lib.hipEventDestroy(e)


def make_weight(torch, t, n, k, gen, dev):
    """Random packed weight with the benchmark distributions, generated on the GPU."""
    qk, bb = BLOCK[t]
    nb = n * (k // qk)
    w = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=dev, generator=gen)

    def f16_field(scale):
        return (torch.randn(nb, device=dev, generator=gen).abs() * scale).half().view(torch.uint8).view(nb, 2)

    if t == Q4_0:
        w[:, 0:2] = f16_field(0.02)
    elif t == Q8_0:
        w[:, 0:2] = f16_field(0.01)
        w[:, 2:34] = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
    elif t == Q4_K:
        w[:, 0:2] = f16_field(0.01)
        w[:, 2:4] = f16_field(0.01)
    else:
        w[:, 208:210] = f16_field(0.01)
    return w.view(-1)


class Workload:
    """Weights, activations and the qmm_gemm_desc list of one step.  Activations and outputs are
    fp16 (the reference API's dtype) unless io == "f32"."""

    def __init__(self, torch, qmm, name, specs_per_layer, layers, M, dev, gen, dominant=None, io="f16"):
        self.torch, self.qmm, self.name, self.M = torch, qmm, name, M
        self.io_dtype = torch.float16 if io == "f16" else torch.float32
        self.io_code = qmm.DTYPE_F16 if io == "f16" else qmm.DTYPE_F32
        self.eb = 2 if io == "f16" else 4  # bytes per activation / output element
        self.weights, self.descs_py = [], []
        self.inputs, self.outputs = {}, {}
        widths = {}
        for specs in specs_per_layer:
            for (_, _, n, k, inp) in specs:
                widths[inp] = k
        for inp, k in widths.items():
            self.inputs[inp] = torch.randn((M, k), device=dev, generator=gen, dtype=torch.float32).to(self.io_dtype)
        self.algo_bytes = 0
        self.weight_bytes = 0
        self.flops = 0
        self.dominant_idx = []
        for layer in range(layers):
            specs = specs_per_layer[layer % len(specs_per_layer)]
            for (pname, t, n, k, inp) in specs:
                w = make_weight(torch, t, n, k, gen, dev)
                self.weights.append(w)
                key = (pname, n)
                if key not in self.outputs:
                    self.outputs[key] = torch.empty((M, n), device=dev, dtype=self.io_dtype)
                if dominant is not None and (t, n, k) == dominant:
                    self.dominant_idx.append(len(self.descs_py))
                self.descs_py.append((t, self.inputs[inp], w, self.outputs[key], n, k))
                self.weight_bytes += weight_bytes(t, n, k)
                self.algo_bytes += weight_bytes(t, n, k) + self.eb * M * (k + n)
                self.flops += 2 * M * n * k
        self.dominant = dominant

    def descs(self, events=None):
        """ctypes array of GemmDesc; `events` maps desc index -> (ev_before, ev_after)."""
        qmm = self.qmm
        arr = (qmm.GemmDesc * len(self.descs_py))()
        for i, (t, a, w, c, n, k) in enumerate(self.descs_py):
            d = arr[i]
            d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = t, a.data_ptr(), self.io_code, w.data_ptr(), \
                c.data_ptr(), self.io_code
            d.M, d.N, d.K = self.M, n, k
            ev = events.get(i) if events else None
            d.ev_before, d.ev_after = (ev if ev else (None, None))
        return arr

    def free(self):
        self.weights.clear()
        self.descs_py.clear()


def run_workload(torch, qmm, hip, wl, steps, warmup, per_step=None):
    """Average ms per step (one qmm_gemm_batch call over all descriptors) and wall seconds.
    With `per_step` (a list), a HIP event is also recorded between steps and each step's duration
    in ms is appended to it (for the median / p95)."""
    stream = torch.cuda.current_stream().cuda_stream
    plain = wl.descs()
    for _ in range(warmup):
        qmm.check(qmm.lib().qmm_gemm_batch(plain, len(plain), stream))
    torch.cuda.synchronize()
    evs = [hip.event() for _ in range(steps + 1)]
    wall0 = time.perf_counter()
    hip.record(evs[0], stream)
    for i in range(steps):
        qmm.check(qmm.lib().qmm_gemm_batch(plain, len(plain), stream))
        hip.record(evs[i + 1], stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = hip.elapsed_ms(evs[0], evs[-1])
    if per_step is not None:
        per_step.extend(hip.elapsed_ms(evs[i], evs[i + 1]) for i in range(steps))
    for e in evs:
        hip.destroy(e)
    return total_ms / steps, wall


def run_dominant(torch, qmm, hip, wl, reps, warmup=2):
    """Average duration of the dominant kernel, the fused gate+up launch: one qmm_gemm_batch call
    per layer with that layer's gate and up descriptors (one launch each, distinct weights),
    all layers back to back between two HIP events on the stream they run on, `reps` times;
    returns (avg_us, launches)."""
    stream = torch.cuda.current_stream().cuda_stream
    idx = wl.dominant_idx
    full = wl.descs()
    pairs = []
    for j in range(0, len(idx) - 1, 2):
        arr = (wl.qmm.GemmDesc * 2)()
        arr[0], arr[1] = full[idx[j]], full[idx[j + 1]]
        pairs.append(arr)

    def one_pass():
        for arr in pairs:
            qmm.check(qmm.lib().qmm_gemm_batch(arr, 2, stream))

    for _ in range(warmup):
        one_pass()
    torch.cuda.synchronize()
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for _ in range(reps):
        one_pass()
    hip.record(b, stream)
    torch.cuda.synchronize()
    ms = hip.elapsed_ms(a, b)
    hip.destroy(a)
    hip.destroy(b)
    return ms * 1e3 / (reps * len(pairs)), reps * len(pairs)


def run_prefill(torch, qmm, hip, gen, dev, steps, warmup):
    """Llama-3-8B prefill GEMMs at M = 512: gate and up (Q4_K 14336 x 4096) and down (Q6_K
    4096 x 14336), each on the f16-MFMA path with fp16 activations (the reference API's dtype) and
    with fp32 activations (adds the f16 conversion pass); TFLOP/s = 2*M*N*K / time per call."""
    M = 512
    stream = torch.cuda.current_stream().cuda_stream
    res = {}
    for name, t, n, k in (("gate_q4_k_14336x4096", Q4_K, 14336, 4096), ("up_q4_k_14336x4096", Q4_K, 14336, 4096),
                          ("down_q6_k_4096x14336", Q6_K, 4096, 14336)):
        w = make_weight(torch, t, n, k, gen, dev)
        x32 = torch.randn((M, k), device=dev, generator=gen)
        for adt, x in (("f16", x32.half()), ("f32", x32)):
            c = torch.empty((M, n), device=dev, dtype=x.dtype)
            dt = qmm.DTYPE_F16 if adt == "f16" else qmm.DTYPE_F32

            def launch():
                qmm.check(qmm.lib().qmm_gemm(t, x.data_ptr(), dt, w.data_ptr(), c.data_ptr(), dt, M, n, k, stream))

            for _ in range(warmup):
                launch()
            torch.cuda.synchronize()
            a, b = hip.event(), hip.event()
            hip.record(a, stream)
            for _ in range(steps):
                launch()
            hip.record(b, stream)
            torch.cuda.synchronize()
            us = hip.elapsed_ms(a, b) * 1e3 / steps
            hip.destroy(a)
            hip.destroy(b)
            tf = 2.0 * M * n * k / (us * 1e-6) / 1e12
            key = f"{name}_a{adt}"
            res[key] = {"us": round(us, 2), "TFLOP/s": round(tf, 1), "frac_f16_peak": round(tf / F16_DENSE_PEAK_TFLOPS, 4)}
            log(f"prefill M=512 {key}: {us:.1f} us, {tf:.1f} TFLOP/s ({tf / F16_DENSE_PEAK_TFLOPS * 100:.1f}% of f16 peak)")
            del c
        # context: the vendor f16 GEMM (torch -> hipBLASLt) on dense f16 weights of the same
        # shape, no dequantization (3.5x more weight bytes than Q4_K)
        w16 = torch.randn((n, k), device=dev, generator=gen, dtype=torch.float16)
        x16 = x32.half()
        for _ in range(warmup):
            _ = x16 @ w16.t()
        torch.cuda.synchronize()
        a, b = hip.event(), hip.event()
        hip.record(a, stream)
        for _ in range(steps):
            _ = x16 @ w16.t()
        hip.record(b, stream)
        torch.cuda.synchronize()
        us = hip.elapsed_ms(a, b) * 1e3 / steps
        hip.destroy(a)
        hip.destroy(b)
        tf = 2.0 * M * n * k / (us * 1e-6) / 1e12
        key = f"{name}_dense_f16_vendor_gemm"
        res[key] = {"us": round(us, 2), "TFLOP/s": round(tf, 1), "frac_f16_peak": round(tf / F16_DENSE_PEAK_TFLOPS, 4)}
        log(f"prefill M=512 {key}: {us:.1f} us, {tf:.1f} TFLOP/s (reference point, dense f16 weights)")
        del w, x32, w16, x16
    # gate and up as one qmm_gemm_batch call: the two descriptors share the activations and run as
    # one launch whose 2 x 14336 output rows fill the GPU with 256 x 256 tiles; fp16 activations and
    # outputs, then fp32 ones (one f16 conversion pass of the shared activations per call)
    n, k = 14336, 4096
    ws = [make_weight(torch, Q4_K, n, k, gen, dev) for _ in range(2)]
    x32 = torch.randn((M, k), device=dev, generator=gen)
    for adt, x in (("f16", x32.half()), ("f32", x32)):
        dt = qmm.DTYPE_F16 if adt == "f16" else qmm.DTYPE_F32
        cs = [torch.empty((M, n), device=dev, dtype=x.dtype) for _ in range(2)]
        arr = (qmm.GemmDesc * 2)()
        for d, w, c in zip(arr, ws, cs):
            d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = Q4_K, x.data_ptr(), dt, w.data_ptr(), c.data_ptr(), dt
            d.M, d.N, d.K = M, n, k
            d.ev_before = d.ev_after = None
        for _ in range(warmup):
            qmm.check(qmm.lib().qmm_gemm_batch(arr, 2, stream))
        torch.cuda.synchronize()
        a, b = hip.event(), hip.event()
        hip.record(a, stream)
        for _ in range(steps):
            qmm.check(qmm.lib().qmm_gemm_batch(arr, 2, stream))
        hip.record(b, stream)
        torch.cuda.synchronize()
        us = hip.elapsed_ms(a, b) * 1e3 / steps
        hip.destroy(a)
        hip.destroy(b)
        tf = 2.0 * 2 * M * n * k / (us * 1e-6) / 1e12
        key = f"gate_up_fused_q4_k_2x14336x4096_a{adt}"
        res[key] = {"us": round(us, 2), "TFLOP/s": round(tf, 1), "frac_f16_peak": round(tf / F16_DENSE_PEAK_TFLOPS, 4)}
        log(f"prefill M=512 {key}: {us:.1f} us, {tf:.1f} TFLOP/s ({tf / F16_DENSE_PEAK_TFLOPS * 100:.1f}% of f16 peak)")
        del cs
    del ws, x32
    return res


def time_gemv(torch, qmm, hip, weights, t, n, k, M, io, reps):
    """Average µs of one qmm_gemm call C[M, n] = A[M, k] @ W^T over `weights` (distinct copies of
    one shape, rotated so the footprint exceeds the MALL), back to back on one stream."""
    stream = torch.cuda.current_stream().cuda_stream
    dt = qmm.DTYPE_F16 if io == "f16" else qmm.DTYPE_F32
    tdt = torch.float16 if io == "f16" else torch.float32
    x = torch.randn((M, k), device=weights[0].device).to(tdt)
    c = torch.empty((M, n), device=weights[0].device, dtype=tdt)

    def call(w):
        qmm.check(qmm.lib().qmm_gemm(t, x.data_ptr(), dt, w.data_ptr(), c.data_ptr(), dt, M, n, k, stream))

    for w in weights:
        call(w)
    torch.cuda.synchronize()
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for i in range(reps):
        call(weights[i % len(weights)])
    hip.record(b, stream)
    torch.cuda.synchronize()
    us = hip.elapsed_ms(a, b) * 1e3 / reps
    hip.destroy(a)
    hip.destroy(b)
    return us


def run_small_m(torch, qmm, hip, gen, dev, Ms=(1, 2, 4, 5, 8, 12, 16, 17, 24, 31)):
    """Small M (prompt chunks of fewer than 32 tokens, src/inference.py:255-286) on the 70B gate
    (Q4_K 28672 x 8192) and down (Q6_K 8192 x 28672) shapes, fp16 I/O: µs per call and algorithmic
    GB/s (weights once + activations + outputs).  M <= 16 runs the GEMV kernels (Q4_K: the v_dot2 GEMV
    at M = 1, the matrix-core GEMV from M = 2; Q6_K: v_dot2 in 4- or 8-row blocks), M >= 17 the 32-row
    MFMA tile."""
    res = {}
    for name, t, n, k, copies in (("gate_q4_k_28672x8192", Q4_K, 28672, 8192, 12),
                                  ("down_q6_k_8192x28672", Q6_K, 8192, 28672, 8)):
        ws = [make_weight(torch, t, n, k, gen, dev) for _ in range(copies)]
        for M in Ms:
            us = time_gemv(torch, qmm, hip, ws, t, n, k, M, "f16", 4 * copies)
            g = (weight_bytes(t, n, k) + 2 * M * (n + k)) / (us * 1e-6) / 1e9
            res[f"{name}_m{M}"] = {"us": round(us, 2), "GB/s": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4)}
            log(f"small-M {name} M={M}: {us:.2f} us, {g:.0f} GB/s")
        del ws
        torch.cuda.empty_cache()
    return res


def run_dequant(torch, qmm, hip, gen, dev, reps=20):
    """Dequantization of one 70B matrix to fp16 (qmm_dequantize): µs per call and algorithmic GB/s
    (packed bytes read + 2 bytes written per weight), on 4 rotated copies."""
    res = {}
    stream = torch.cuda.current_stream().cuda_stream
    for name, t, n, k in (("gate_q4_k_28672x8192", Q4_K, 28672, 8192), ("down_q6_k_8192x28672", Q6_K, 8192, 28672)):
        ws = [make_weight(torch, t, n, k, gen, dev) for _ in range(4)]
        out = torch.empty(n * k, device=dev, dtype=torch.float16)

        def call(w):
            qmm.check(qmm.lib().qmm_dequantize(t, w.data_ptr(), out.data_ptr(), qmm.DTYPE_F16, n * k, stream))

        for w in ws:
            call(w)
        torch.cuda.synchronize()
        a, b = hip.event(), hip.event()
        hip.record(a, stream)
        for i in range(reps):
            call(ws[i % len(ws)])
        hip.record(b, stream)
        torch.cuda.synchronize()
        us = hip.elapsed_ms(a, b) * 1e3 / reps
        hip.destroy(a)
        hip.destroy(b)
        nbytes = weight_bytes(t, n, k) + 2 * n * k
        g = nbytes / (us * 1e-6) / 1e9
        res[f"{name}_to_f16"] = {"us": round(us, 2), "bytes": nbytes, "GB/s": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4)}
        log(f"dequant {name} -> f16: {us:.1f} us, {g:.0f} GB/s")
        del ws, out
        torch.cuda.empty_cache()
    return res


# Time per call at the target fraction of peak (GEMV 70 % of HBM, prefill 50 % of the dense f16 peak)
TARGETS_US = {"8b_q8_0_layer_m1": 41.4, "8b_q4_k_m_layer_m1": 24.7, "8b_q6_k_lm_head_m1": 77.0,
              "prefill_m512_per_matrix": 47.8, "70b_q4_k_m_layer_m1": 96.9, "70b_q4_k_m_layer_m4": 97.2}


def run_full_layers(torch, qmm, hip, wl, layers, proj_ms, dev, gen, steps, context=1024):
    """Whole Llama-3-70B layers (qmm_forward_layer: RMSNorm, q/k/v, RoPE + KV write, attention
    over the cache, o, residual + RMSNorm, gate/up, SwiGLU, down, residual) on the decode
    benchmark's 80 resident Q4_K_M layers: a (context - 1)-token prefill through all layers fills
    the KV cache (timed: prefill tokens/s), then decode steps of one token at position
    context - 1 attend over `context` keys (timed: ms per token), beside the projections-only
    step of the same weights."""
    hidden, inter, heads, kvh, d = 8192, 28672, 64, 8, 128
    c = qmm.LayerConfig()
    c.hidden_size, c.intermediate_size, c.num_heads, c.num_kv_heads, c.head_dim = hidden, inter, heads, kvh, d
    c.rms_norm_eps, c.rope_freq_base, c.rope_neox, c.scale = 1e-5, 500000.0, 0, 0.0
    norm = torch.ones(hidden, dtype=torch.float16, device=dev)
    ws = []
    for layer in range(layers):
        w = qmm.LayerWeights()
        w.attn_norm, w.attn_norm_dtype, w.ffn_norm, w.ffn_norm_dtype = norm.data_ptr(), qmm.DTYPE_F16, norm.data_ptr(), \
            qmm.DTYPE_F16
        for i, f in enumerate(("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")):
            t, _, wt, _, _, _ = wl.descs_py[7 * layer + i]
            setattr(w, f, wt.data_ptr())
            setattr(w, f + "_type", t)
        ws.append(w)
    stream = torch.cuda.current_stream().cuda_stream
    lib = qmm.lib()
    qmm.check(lib.qmm_kv_cache_init(layers, context, kvh, d))
    try:
        P = context - 1
        xa = (torch.randn((P, hidden), device=dev, generator=gen) * 0.5).half()
        xb = torch.empty_like(xa)

        def prefill():
            a, b = xa, xb
            for layer in range(layers):
                qmm.check(lib.qmm_forward_layer(c, ws[layer], a.data_ptr(), b.data_ptr(), layer, P, 0, stream))
                a, b = b, a

        prefill()  # warm-up (workspace growth, first touch)
        torch.cuda.synchronize()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        prefill()
        hip.record(e1, stream)
        torch.cuda.synchronize()
        pre_ms = hip.elapsed_ms(e0, e1)
        ya, yb = xa[:1].clone(), xa[:1].clone()

        def decode():
            a, b = ya, yb
            for layer in range(layers):
                qmm.check(lib.qmm_forward_layer(c, ws[layer], a.data_ptr(), b.data_ptr(), layer, 1, P, stream))
                a, b = b, a

        decode()
        torch.cuda.synchronize()
        hip.record(e0, stream)
        for _ in range(steps):
            decode()
        hip.record(e1, stream)
        torch.cuda.synchronize()
        dec_ms = hip.elapsed_ms(e0, e1) / steps
        hip.destroy(e0)
        hip.destroy(e1)
    finally:
        qmm.check(lib.qmm_kv_cache_free())
        qmm.check(lib.qmm_release_workspace())
    res = {"layers": layers, "context": context, "decode_ms_per_token": round(dec_ms, 3),
           "decode_tokens_per_s": round(1e3 / dec_ms, 1), "projections_only_ms_per_token": round(proj_ms, 3),
           "prefill_tokens": P, "prefill_ms": round(pre_ms, 2), "prefill_tokens_per_s": round(P / (pre_ms * 1e-3), 1),
           "note": "whole layers; weights of the decode benchmark; fp16 activations; embedding and lm_head excluded"}
    log(f"70B full layers: decode {dec_ms:.3f} ms/token at context {context} (projections alone {proj_ms:.3f}); "
        f"prefill {P} tokens {pre_ms:.1f} ms = {res['prefill_tokens_per_s']} tokens/s")
    return res


def run_upload(torch, qmm, dev, layers=2):
    """Weight residency: a GGUF file holding `layers` Llama-3-70B Q4_K_M layers (7 packed
    matrices each, 542 MB per layer, random bytes) is loaded into HBM from the page cache
    (the file was just written) by resident.ResidentWeights (qmm_upload_file: parallel pread
    into pinned staging buffers overlapped with host -> device copies), and, as the reference
    path does it, by copying each tensor's mmap view to the device from pageable memory."""
    import mmap
    import tempfile

    import numpy as np

    import gguf
    import resident

    rng = np.random.default_rng(5)
    tensors = []
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
             "down": "ffn_down"}
    for i in range(layers):
        for (nm, t, n, k, _) in layer_specs(8192, 28672, 1024, Q4_K, Q6_K):
            nbytes = weight_bytes(t, n, k)
            tensors.append((f"blk.{i}.{names[nm]}.weight", (k, n), gguf.GGMLType(t), rng.bytes(nbytes)))
    meta = {"general.architecture": (gguf.GGUFValueType.STRING, "llama"),
            "llama.block_count": (gguf.GGUFValueType.UINT32, layers)}
    fd, path = tempfile.mkstemp(suffix=".gguf")
    try:
        with os.fdopen(fd, "wb") as f:
            gguf.write_synthetic_gguf(f, meta, tensors)
        del tensors
        total = os.path.getsize(path)
        res = {"file_GB": round(total / 1e9, 3)}
        for rep in range(2):  # the first load also pays the allocator's first touch
            torch.cuda.synchronize()
            rw = resident.ResidentWeights(path, device=dev)
            nbytes, secs = rw.nbytes, rw.upload_seconds
            rw.close()
            del rw
            torch.cuda.empty_cache()
        res["resident_GB/s"] = round(nbytes / secs / 1e9, 2)
        res["resident_s"] = round(secs, 3)
        p = resident.parse_file(path)
        with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            outs = []
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for t in p.tensors.values():
                view = np.frombuffer(mm, dtype=np.uint8, count=t.n_bytes, offset=t.abs_offset)
                outs.append(torch.from_numpy(view).to(dev))
            torch.cuda.synchronize()
            secs = time.perf_counter() - t0
            del outs, view
        res["pageable_mmap_copy_GB/s"] = round(nbytes / secs / 1e9, 2)
        res["note"] = ("page-cache -> HBM over the host link (PCIe 5.0 x16: 64 GB/s per direction); "
                       "pageable = per-tensor torch copy of the mmap view, the reference's route")
        torch.cuda.empty_cache()
        log(f"weight upload ({total / 1e9:.2f} GB GGUF): resident {res['resident_GB/s']} GB/s, "
            f"pageable mmap copy {res['pageable_mmap_copy_GB/s']} GB/s")
        return res
    finally:
        os.unlink(path)


def cpu_host_info():
    """CPU model (/proc/cpuinfo), usable cores and the BLAS thread pools actually loaded."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas = []
    try:
        from threadpoolctl import threadpool_info

        blas = [f"{i.get('internal_api')}:{i.get('num_threads')}" for i in threadpool_info() if i.get("user_api") == "blas"]
    except Exception:  # threadpoolctl absent: report the environment instead
        blas = [f"env:{os.environ.get('OPENBLAS_NUM_THREADS') or os.environ.get('OMP_NUM_THREADS') or 'default'}"]
    return {"cpu_model": model, "cores": len(os.sched_getaffinity(0)), "blas_threads": ",".join(blas) or "none"}


def _median(v):
    v = sorted(v)
    return v[len(v) // 2]


def cpu_config(O, np, mats, Ms, rng, frac, reps):
    """The reference CPU path on one configuration: per matrix, NumPy dequantization to fp16
    (src/gguf_parser.py:374-589) timed on a sample of its rows and scaled to all rows (the
    dequantizer's cost is linear in the rows), then `A.astype(f32) @ W.astype(f32).T`
    (tests/test_gguf_and_q4.py:127-128) timed at full size for each M in `Ms` on a matrix tiled
    from the sampled rows.  Each timing is the median of `reps` runs after one warm-up run.
    Returns (dequant seconds, {M: matmul seconds}, packed weight bytes)."""
    deq_s = 0.0
    mm_s = {M: 0.0 for M in Ms}
    wbytes = 0
    for (_, t, n, k) in mats:
        ns = max(1, int(round(n * frac)))
        raw = O.synth_weights(t, ns, k, rng)
        times = []
        for _ in range(reps + 1):
            t0 = time.perf_counter()
            w16 = O.dequantize_f16(t, raw, ns * k)
            times.append(time.perf_counter() - t0)
        deq_s += _median(times[1:]) * n / ns
        full = np.tile(w16.reshape(ns, k), (-(-n // ns), 1))[:n]
        for M in Ms:
            a = rng.standard_normal((M, k)).astype(np.float32)
            times = []
            for _ in range(reps + 1):
                t0 = time.perf_counter()
                _ = a.astype(np.float32) @ full.astype(np.float32).T
                times.append(time.perf_counter() - t0)
            mm_s[M] += _median(times[1:])
        wbytes += weight_bytes(t, n, k)
        del full, raw, w16
    return deq_s, mm_s, wbytes


def cpu_baseline(seed=0):
    """The in-repo NumPy restatement of the reference's CPU path, timed on the host cores beside
    the GPU for every benchmark configuration (dequantization and GEMV/GEMM reported separately;
    dequantization sampled on a fraction of each matrix's rows and scaled, the matmul at full
    size).  The headline object is the 70B Q4_K_M layer at M = 1 (one layer, extrapolated to 80)."""
    import numpy as np

    import gguf_oracle as O

    rng = np.random.default_rng(seed)
    info = cpu_host_info()
    t_start = time.perf_counter()

    def mats(specs):
        return [(name, t, n, k) for (name, t, n, k, _) in specs]

    configs = {  # key: (matrices, M values, dequant row sample, timed runs)
        "c1_q4_0_4096x4096": ([("w", Q4_0, 4096, 4096)], (1,), 1.0, 5),
        "c2_8b_q8_0_layer": (mats(layer_specs(4096, 14336, 1024, Q8_0, Q8_0)), (1,), 1 / 8, 3),
        "c3_8b_q4_k_m_layer": (mats(layer_specs(4096, 14336, 1024, Q4_K, Q6_K)), (1,), 1 / 8, 3),
        "c3_8b_q6_k_lm_head": ([("lm_head", Q6_K, 128256, 4096)], (1,), 1 / 64, 2),
        "c4_8b_prefill": ([("gate", Q4_K, 14336, 4096), ("up", Q4_K, 14336, 4096), ("down", Q6_K, 4096, 14336)],
                          (512,), 1 / 8, 3),
        "c5_70b_q4_k_m_layer": (mats(layer_specs(8192, 28672, 1024, Q4_K, Q6_K)), (1, 4), 1 / 64, 2),
    }
    res = {}
    for key, (ms_, Ms, frac, reps) in configs.items():
        deq, mm, wb = cpu_config(O, np, ms_, Ms, rng, frac, reps)
        for M in Ms:
            tot = deq + mm[M]
            r = {"dequant_s": round(deq, 4), "matmul_s": round(mm[M], 4), "total_s": round(tot, 4),
                 "dequant_row_sample": round(frac, 4), "timed_runs": reps}
            if key.startswith("c4"):
                flops = sum(2 * M * n * k for (_, _, n, k) in ms_)
                r["TFLOP/s"] = round(flops / tot / 1e12, 4)
                r["matmul_only_TFLOP/s"] = round(flops / mm[M] / 1e12, 4)
            else:
                nbytes = wb + 4 * M * sum(k + n for (_, _, n, k) in ms_)
                r["GB/s"] = round(nbytes / tot / 1e9, 4)
            if key.startswith("c5"):
                r["ms_per_token_extrapolated_80_layers"] = round(tot * 80 * 1e3, 1)
            res[f"{key}_m{M}"] = r
            log(f"cpu {key} M={M}: {r}")
    head = res["c5_70b_q4_k_m_layer_m1"]
    return {
        "value": head["GB/s"],
        "unit": "GB/s",
        "cores": info["cores"],
        "kind": "port",
        "sample": ("one Llama-3-70B Q4_K_M layer (7 matrices, 542 MB packed), M=1, fp32 activations: NumPy "
                   "dequantize to fp16 (single thread) timed on 1/64 of each matrix's rows and scaled, then fp32 "
                   "matmul (BLAS) at full size; median of 2 after a warm-up; 80-layer time extrapolated"),
        "cpu_model": info["cpu_model"],
        "blas_threads": info["blas_threads"],
        "configs": res,
        "wall_s": round(time.perf_counter() - t_start, 1),
    }


def pmc_workload(torch, qmm, dev, gen, reps=8):
    """Counter-collection workload: a plain device copy of known size (256 MiB read + 256 MiB
    written per launch), then the dominant kernel (fused gate+up: two Q4_K 28672 x 8192 GEMVs on
    one activation vector, M = 1) over 8 distinct weight pairs.  Run under `rocprofv3 --pmc
    FETCH_SIZE` and `--pmc WRITE_SIZE`: the copy's per-dispatch reading calibrates the counter
    against known bytes."""
    stream = torch.cuda.current_stream().cuda_stream
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    n, k = 28672, 8192
    ws = [make_weight(torch, Q4_K, n, k, gen, dev) for _ in range(16)]
    x = torch.randn((1, k), device=dev, generator=gen).half()
    ys = [torch.empty((1, n), device=dev, dtype=torch.float16) for _ in range(2)]
    pairs = []
    for j in range(0, 16, 2):
        arr = (qmm.GemmDesc * 2)()
        for e in range(2):
            d = arr[e]
            d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = (Q4_K, x.data_ptr(), qmm.DTYPE_F16, ws[j + e].data_ptr(),
                                                                ys[e].data_ptr(), qmm.DTYPE_F16)
            d.M, d.N, d.K = 1, n, k
        pairs.append(arr)
    for r in range(reps):
        for arr in pairs:
            qmm.check(qmm.lib().qmm_gemm_batch(arr, 2, stream))
    torch.cuda.synchronize()
    log(f"pmc workload done: copy 256 MiB x {reps}, fused gate+up (2 x Q4_K {n}x{k}) x {8 * reps}")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=80)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the prefill section (8B M=512 shapes) and print its results as JSON")
    ap.add_argument("--full-layers-only", action="store_true",
                    help="run only the whole-layer 70B section (prefill through the KV cache, then decode) and "
                         "print its results as JSON")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run only the counter-collection workload (copy calibration + dominant GEMV)")
    ap.add_argument("--small-m-only", action="store_true",
                    help="run only the small-M (70B gate / down at M = 1..31) and dequantize sections and print "
                         "their results as JSON")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; only one GPU is measured "
              "(the path would shard by weight rows, one slice per GPU).", file=sys.stderr)
        sys.exit(2)

    import torch

    import qmm

    dev = torch.device("cuda:0")
    hip = Hip()
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")
    if args.pmc_workload:
        pmc_workload(torch, qmm, dev, gen)
        return
    if args.small_m_only:
        print(json.dumps({"70b_small_m": run_small_m(torch, qmm, hip, gen, dev),
                          "dequant_70b": run_dequant(torch, qmm, hip, gen, dev)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill_8b_m512": run_prefill(torch, qmm, hip, gen, dev, max(3, args.steps // 2), 2)}),
              flush=True)
        return

    # ---- headline: Llama-3-70B Q4_K_M, M=1, 80 distinct layers -----------------------------
    t0 = time.perf_counter()
    specs70 = layer_specs(8192, 28672, 1024, Q4_K, Q6_K)
    dominant = (Q4_K, 28672, 8192)
    wl = Workload(torch, qmm, "70b", [specs70], args.layers, 1, dev, gen, dominant=dominant)
    torch.cuda.synchronize()
    log(f"70B weights ready: {wl.weight_bytes / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
    if args.full_layers_only:
        ms, _ = run_workload(torch, qmm, hip, wl, max(3, args.steps // 2), 2)
        print(json.dumps({"70b_q4_k_m_full_layers": run_full_layers(torch, qmm, hip, wl, args.layers, ms, dev, gen,
                                                                    max(3, args.steps // 2))}), flush=True)
        return
    step_ms = []
    ms, wall = run_workload(torch, qmm, hip, wl, args.steps, args.warmup, per_step=step_ms)
    step_ms.sort()
    p50 = step_ms[len(step_ms) // 2]
    p95 = step_ms[min(len(step_ms) - 1, int(round(0.95 * (len(step_ms) - 1))))]
    gbs = wl.algo_bytes / (ms * 1e-3) / 1e9
    log(f"70B M=1: {ms:.3f} ms/token (median {p50:.3f}, p95 {p95:.3f}), {gbs:.1f} GB/s "
        f"({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM peak), wall {wall:.3f} s for {args.steps} steps")
    dom_bytes = 2 * weight_bytes(Q4_K, 28672, 8192) + wl.eb * (8192 + 2 * 28672)
    dom_us, dom_launches = run_dominant(torch, qmm, hip, wl, max(2, args.steps // 4))
    dom_gbs = dom_bytes / (dom_us * 1e-6) / 1e9
    log(f"dominant kernel (fused gate+up, 2 x Q4_K 28672x8192 GEMV, M=1): {dom_us:.2f} us avg over "
        f"{dom_launches} back-to-back launches, {dom_gbs:.1f} GB/s")

    traffic = read_traffic()

    extra = {}
    if not args.no_extra:
        # 70B at M = 4 on the same resident weights.
        wl4 = Workload.__new__(Workload)
        wl4.__dict__.update(wl.__dict__)
        wl4.M = 4
        wl4.inputs = {k: torch.randn((4, v.shape[1]), device=dev, generator=gen).to(wl.io_dtype)
                      for k, v in wl.inputs.items()}
        wl4.outputs = {k: torch.empty((4, v.shape[1]), device=dev, dtype=wl.io_dtype) for k, v in wl.outputs.items()}
        remap_in = {id(wl.inputs[k]): wl4.inputs[k] for k in wl.inputs}
        remap_out = {id(wl.outputs[k]): wl4.outputs[k] for k in wl.outputs}
        wl4.descs_py = [(t, remap_in[id(a)], w, remap_out[id(c)], n, k) for (t, a, w, c, n, k) in wl.descs_py]
        wl4.algo_bytes = sum(weight_bytes(t, n, k) + 4 * wl.eb * (k + n) for (t, _, _, _, n, k) in wl4.descs_py)
        ms4, _ = run_workload(torch, qmm, hip, wl4, max(3, args.steps // 2), 2)
        extra["70b_q4_k_m_m4"] = {"GB/s": round(wl4.algo_bytes / (ms4 * 1e-3) / 1e9, 1), "ms_per_token": round(ms4, 3),
                                  "frac_hbm": round(wl4.algo_bytes / (ms4 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                  "us_per_layer": round(ms4 * 1e3 / args.layers, 2),
                                  "target_us_per_layer_at_70pct": TARGETS_US["70b_q4_k_m_layer_m4"]}
        log(f"70B M=4: {ms4:.3f} ms/step, {extra['70b_q4_k_m_m4']['GB/s']} GB/s")
    if not args.no_extra:
        extra["70b_q4_k_m_full_layers"] = run_full_layers(torch, qmm, hip, wl, args.layers, ms, dev, gen,
                                                          max(3, args.steps // 2))
    wl.free()
    del wl
    torch.cuda.empty_cache()

    if not args.no_extra:
        # 8B layers rotated over enough copies to exceed the 256 MB MALL (>= 1.8 GB).
        for key, main_t, down_t, copies, io in (("8b_q8_0_layer_m1", Q8_0, Q8_0, 8, "f16"),
                                                 ("8b_q8_0_layer_m1_af32", Q8_0, Q8_0, 8, "f32"),
                                                 ("8b_q4_k_m_layer_m1", Q4_K, Q6_K, 14, "f16")):
            w8 = Workload(torch, qmm, key, [layer_specs(4096, 14336, 1024, main_t, down_t)], copies, 1, dev, gen, io=io)
            ms8, _ = run_workload(torch, qmm, hip, w8, args.steps, args.warmup)
            per_layer_us = ms8 * 1e3 / copies
            g = w8.algo_bytes / (ms8 * 1e-3) / 1e9
            extra[key] = {"GB/s": round(g, 1), "us_per_layer": round(per_layer_us, 2), "frac_hbm": round(g / HBM_PEAK_GBS, 4),
                          "target_us_at_70pct": TARGETS_US.get(key.replace("_af32", "")),
                          "io": io, "tokens_per_s_equiv_32_layers": round(1e6 / (per_layer_us * 32), 1),
                          "footprint_GB": round(w8.weight_bytes / 1e9, 2)}
            log(f"{key}: {extra[key]}")
            w8.free()
            del w8
            torch.cuda.empty_cache()
        extra["8b_prefill_m512"] = run_prefill(torch, qmm, hip, gen, dev, max(3, args.steps // 2), 2)
        extra["8b_prefill_m512"]["target_us_per_matrix_at_50pct"] = TARGETS_US["prefill_m512_per_matrix"]
        torch.cuda.empty_cache()
        extra["70b_small_m"] = run_small_m(torch, qmm, hip, gen, dev)
        extra["dequant_70b"] = run_dequant(torch, qmm, hip, gen, dev)
        torch.cuda.empty_cache()
        lm = Workload(torch, qmm, "lm_head", [[("lm_head", Q6_K, 128256, 4096, "h")]], 4, 1, dev, gen)
        msl, _ = run_workload(torch, qmm, hip, lm, args.steps, args.warmup)
        g = lm.algo_bytes / (msl * 1e-3) / 1e9
        extra["8b_q6_k_lm_head_m1"] = {"GB/s": round(g, 1), "us": round(msl * 1e3 / 4, 2), "frac_hbm": round(g / HBM_PEAK_GBS, 4),
                                       "target_us_at_70pct": TARGETS_US["8b_q6_k_lm_head_m1"]}
        log(f"lm_head: {extra['8b_q6_k_lm_head_m1']}")
        # token embeddings gathered and dequantized from the same Q6_K 128256 x 4096 table
        # (the reference does this on the CPU, src/tokenizer.py:336-389)
        table = lm.weights[0]
        stream = torch.cuda.current_stream().cuda_stream
        for label, ntok in (("prompt_512", 512), ("decode_1", 1)):
            ids = torch.randint(0, 128256, (ntok,), device=dev, generator=gen, dtype=torch.int64)
            out = torch.empty((ntok, 4096), device=dev, dtype=torch.float16)

            def emb():
                qmm.check(qmm.lib().qmm_embed(Q6_K, table.data_ptr(), 128256, 4096, ids.data_ptr(), ntok,
                                              out.data_ptr(), qmm.DTYPE_F16, None, stream))

            for _ in range(3):
                emb()
            torch.cuda.synchronize()
            a, b = hip.event(), hip.event()
            hip.record(a, stream)
            for _ in range(50):
                emb()
            hip.record(b, stream)
            torch.cuda.synchronize()
            us = hip.elapsed_ms(a, b) * 1e3 / 50
            hip.destroy(a)
            hip.destroy(b)
            nbytes = ntok * (weight_bytes(Q6_K, 1, 4096) + 8 + 2 * 4096)
            extra[f"8b_q6_k_embed_{label}"] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1)}
            log(f"embed {label}: {extra[f'8b_q6_k_embed_{label}']}")
        lm.free()
        del lm
        q40 = Workload(torch, qmm, "q4_0", [[("w", Q4_0, 4096, 4096, "h")]], 128, 1, dev, gen, io="f32")
        msq, _ = run_workload(torch, qmm, hip, q40, args.steps, args.warmup)
        g = q40.algo_bytes / (msq * 1e-3) / 1e9
        extra["q4_0_4096x4096_m1"] = {"GB/s": round(g, 1), "us": round(msq * 1e3 / 128, 2),
                                      "note": "128 distinct copies (1.2 GB) streamed back to back"}
        log(f"q4_0: {extra['q4_0_4096x4096_m1']}")
        q40.free()
        del q40
        torch.cuda.empty_cache()
        extra["gguf_weight_upload_70b_2_layers"] = run_upload(torch, qmm, dev)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (NumPy restatement of the reference CPU path) ...")
        cpu = cpu_baseline()
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} cores")

    line = {
        "metric": "Q4_K/Q6_K GEMV GB/s (% of HBM peak) at 8B/70B shapes; prefill TFLOP/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "dtype_detail": "fp16 activations and outputs (the reference API's dtype); Q4_K/Q6_K codes as exact "
                        "f16; f16 x f16 products (v_dot2_f32_f16) accumulated in fp32",
        "data": "synthetic: random packed blocks (fp16 scales |N(0,1)|*0.01), x ~ N(0,1)",
        "config": {"workload": "llama3-70b-q4_k_m-decode-m1-80-layers", "layers": args.layers, "M": 1,
                   "hidden": 8192, "intermediate": 28672, "kv_dim": 1024,
                   "weights_GB": round(wl_bytes_gb(args.layers), 2), "gemvs_per_step": 7 * args.layers,
                   "launches_per_step": 4 * args.layers,
                   "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                   "tokens_per_s": round(1e3 / ms, 1),
                   "ms_per_token_p50": round(p50, 4), "ms_per_token_p95": round(p95, 4),
                   "target_ms_per_token_at_70pct": 7.75},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "gemv_resident_kernel<GQ4K, M=1>, fused gate+up (2 x Q4_K 28672x8192)",
                     "avg_us": round(dom_us, 3), "launches": dom_launches,
                     "algorithmic_bytes_per_launch": dom_bytes},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


TRAFFIC_FILE = os.path.join(REPO, "profiles", "gemv_q4_k_gate_up_2x28672x8192_m1_traffic.md")


def read_traffic():
    """HBM bytes per launch of the dominant kernel from its committed counter summary (the
    `hbm_bytes_per_launch:` line), or None when the summary is absent."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            if line.strip().startswith("hbm_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    return None


def wl_bytes_gb(layers):
    s = layer_specs(8192, 28672, 1024, Q4_K, Q6_K)
    return layers * sum(weight_bytes(t, n, k) for (_, t, n, k, _) in s) / 1e9


if __name__ == "__main__":
    main()
