"""Benchmark of the DP-SGD hot path on one MI355X.

Default workload ("cfg2"): the clipped per-sample weight
gradient of a DP Linear 768 -> 3072 in bf16 with x [8,1024,768] ~ N(0,1),
grad_out [8,1024,3072] ~ N(0,0.02^2), C = 1, sigma = 1:
    dW = (1/B) sum_b clip(||g_b^T x_b||) g_b^T x_b + (sigma/sqrt(B)) z
One step = one fdp_wgrad_clip call, which is one launch of the single-pass
kernel: per-sample products, norms, factors, clipped sum, 1/B, and the
Gaussian noise drawn (Philox4x32-10) and added in its epilogue; inputs
resident in HBM, default (ordinary-dispatch) launch.

value = algorithmic TFLOP/s = 2*B*T*M*N / step time (norm, scale and recompute
flops are not credited).  The JSON line also carries the roofline of the
dominant kernel (its mean duration from a pair of HIP events around every call
of the timed region, on the launch stream; one call is one launch), the host
time per call, the reference's torch op sequence timed on the host CPU
(cpu_baseline, bf16 and fp32), and extra measurements: the same step with the
cooperative launch, the DP Linear layer fwd+bwd vs a plain nn.Linear, the
Conv1D (cfg3) and LayerNorm (cfg4) paths, and DP vs non-DP training tokens/s of
the cfg5 decoder.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2|cfg3|cfg4]
                       [--single-pass auto|unpaired|narrow] [--no-cpu-baseline]
                       [--no-extra] [--copy-calibration MiB]

--single-pass picks the kernel of the cfg2/cfg3 step as wgrad_clip's argument
of that name does (default auto: at cfg2 the paired wide kernel); the
profiles of the other kernels are made with it.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

# HBM bytes per launch of the dominant kernel, from rocprofv3 --pmc FETCH_SIZE
# and WRITE_SIZE runs of this script (the HBM traffic sections of profiles/*.md), each scaled by the
# factor the same counter reads on a plain copy of known size.  None = not
# measured for that workload.
TRAFFIC_BYTES = {  # (workload, --single-pass)
    ("cfg2", "auto"): 109053575,      # profiles/wgrad_pair_kernel_cfg2.md
    ("cfg2", "unpaired"): 134239518,  # profiles/wgrad_wide_kernel_cfg2.md
    ("cfg3", "auto"): 233419812,     # profiles/wgrad_group_kernel_cfg3.md (weight and bias)
    ("cfg4", "auto"): 105565315,     # profiles/layernorm_bwd_clip_cfg4.md (one launch per call)
}
# the dominant kernel of each (workload, --single-pass)
KERNELS = {
    ("cfg2", "auto"): "wgrad_pair_kernel (two samples' 192x192 tiles per CU)",
    ("cfg2", "unpaired"): "wgrad_wide_kernel (one sample's 384x192 tile per CU)",
    ("cfg2", "narrow"): "wgrad_group_kernel (128x128 tiles)",
    ("cfg3", "auto"): "wgrad_group_kernel (weight and bias)",
    ("cfg3", "narrow"): "wgrad_group_kernel (weight and bias)",
}


def cuda_time(fn, steps, warmup, stream=None):
    """Average ms per call of fn over `steps` back-to-back calls, HIP events on the
    current stream (the stream every kernel here is launched on)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def median_cuda_time(fn, steps, warmup, reps=5):
    return statistics.median(cuda_time(fn, steps, warmup if i == 0 else 1) for i in range(reps))


# ------------------------------------------------------------------ workloads
def cfg2_inputs(dev):
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(8, 1024, 768, device=dev, generator=g).to(torch.bfloat16)
    go = (torch.randn(8, 1024, 3072, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w = (torch.randn(3072, 768, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    return x, go, w


def cfg3_inputs(dev):
    """Conv1D c_attn 768 -> 2304, B=16, T=1024, per-sample norms 0.1C..10C."""
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(16, 1024, 768, device=dev, generator=g).to(torch.bfloat16)
    gh = torch.randn(16, 1024, 2304, device=dev, generator=g) * 0.02
    from flashdp4review_amd.core import wgrad_clip
    _, n, _ = wgrad_clip(x, gh.to(torch.bfloat16), 1e30, 1.0, return_stats=True)
    u = torch.rand(16, device=dev, generator=g) * 2 - 1
    go = (gh * ((10.0 ** u) / n)[:, None, None]).to(torch.bfloat16)
    return x, go


def run_wgrad(x, go, out_dtype, sigma=1.0, transpose=False, launch=None, single_pass="auto",
              bias=False):
    """One DP weight-gradient step: the fused clipped product sum with its noise
    drawn in the epilogue (a fresh Philox counter range every step).  With
    `bias`, the layer's bias gradient (column sums of grad_output, clipped by
    ||g_b||, mean over B*T, noise) in the same call, as the DP layers run it
    (transpose: the Conv1D orientation x^T g, whose bias is of operand b)."""
    from flashdp4review_amd.core import wgrad_clip
    from flashdp4review_amd.layers.utils import NoiseStream
    B, T = x.shape[0], x.shape[1]
    a, b = (x, go) if transpose else (go, x)
    M, N = a.shape[2], b.shape[2]
    std = sigma / math.sqrt(B)
    keys = NoiseStream()
    O = go.shape[2]
    bias_out = torch.empty(O, dtype=go.dtype, device=go.device) if bias else None

    def step():
        kw = {}
        if bias:
            kw = dict(bias_out=bias_out, bias_scale=1.0 / (B * T), bias_noise_scale=std,
                      bias_noise_key=keys.next(O), bias_operand="b" if transpose else "a")
        return wgrad_clip(a, b, 1.0, 1.0, layout="tn", out_scale=1.0 / B, noise_scale=std,
                          noise_key=keys.next(M * N), out_dtype=out_dtype, launch=launch,
                          single_pass=single_pass, **kw)

    return step, step


# --------------------------------------------------------------- cpu baseline
def host_cores():
    """Cores this process may run on (its CPU affinity set), and the machine's count."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        avail = os.cpu_count() or 1
    return avail, os.cpu_count() or avail


def _cpu_leg(dtype, budget_s):
    """Median seconds per cfg2 step of the reference's torch op sequence in `dtype`."""
    from oracle import torch_ref
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 1024, 768, generator=g).to(dtype)
    go = (torch.randn(8, 1024, 3072, generator=g) * 0.02).to(dtype)
    torch_ref.linear_weight_backward(x, go, 1.0, 1.0, 1.0)  # warm-up
    ts = []
    t_start = time.perf_counter()
    while len(ts) < 3 or (time.perf_counter() - t_start < budget_s and len(ts) < 500):
        t0 = time.perf_counter()
        torch_ref.linear_weight_backward(x, go, 1.0, 1.0, 1.0)
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


def _timed(fn, budget_s):
    """Median seconds per call of fn after one warm-up (at least 3 calls)."""
    fn()
    ts = []
    t_start = time.perf_counter()
    while len(ts) < 3 or (time.perf_counter() - t_start < budget_s and len(ts) < 500):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


def cpu_baselines_cfg3_cfg4(budget_s=4.0):
    """The reference's torch path on the host cores for cfg3 (Conv1D weight
    gradient x^T g with the bias clip, flashdp/core/transformers_conv1d_clip.py:22-39
    via the same per-sample op sequence) and cfg4 (LayerNorm backward with the
    per-sample dgamma/dbeta clip and noise, flashdp/layers/layernorm.py:92-155),
    full batches, in bf16 (the config dtype) and fp32."""
    from oracle import torch_ref
    threads, machine = host_cores()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    out = {}
    try:
        g = torch.Generator().manual_seed(0)
        res3 = {}
        for dt in (torch.bfloat16, torch.float32):
            x = torch.randn(16, 1024, 768, generator=g).to(dt)
            go = (torch.randn(16, 1024, 2304, generator=g) * 0.02).to(dt)

            def step3():
                torch_ref.linear_weight_backward(go, x, 1.0, 1.0, 1.0)  # x^T g: [768, 2304]
                torch_ref.linear_bias_grad_clip(go.clone(), 1.0, 1.0)
            t, n = _timed(step3, budget_s)
            res3[str(dt).split(".")[1]] = (t, n)
        F3 = 2.0 * 16 * 1024 * 768 * 2304
        out["cpu_cfg3"] = {"value": round(F3 / res3["bfloat16"][0] / 1e12, 4), "unit": "TFLOP/s",
                           "fp32_value": round(F3 / res3["float32"][0] / 1e12, 4),
                           "cores": threads, "kind": "port",
                           "sample": "cfg3 full batch (B=16,T=1024, Conv1D 768->2304) on CPU: "
                                     "clipped dW + noise and the clipped bias, median step: bf16 "
                                     f"{res3['bfloat16'][0]:.4f} s over {res3['bfloat16'][1]} "
                                     f"steps, fp32 {res3['float32'][0]:.4f} s over "
                                     f"{res3['float32'][1]} steps"}
        res4 = {}
        for dt in (torch.bfloat16, torch.float32):
            x = torch.randn(16, 1024, 1024, generator=g).to(dt)
            go = (torch.randn(16, 1024, 1024, generator=g) * 0.01).to(dt)
            w = torch.ones(1024, dtype=dt)
            t, n = _timed(lambda: torch_ref.layernorm_backward(x, w, go, 1e-5, 1.0, 1.0, 1.0),
                          budget_s)
            res4[str(dt).split(".")[1]] = (t, n)
        nbytes = 3 * 2 * 16 * 1024 * 1024 + 8 * 16 * 1024
        out["cpu_cfg4"] = {"value": round(nbytes / res4["bfloat16"][0] / 1e9, 2), "unit": "GB/s",
                           "fp32_value": round(nbytes / res4["float32"][0] / 1e9, 2),
                           "cores": threads, "kind": "port",
                           "sample": "cfg4 full batch (B=16,T=1024,H=1024) on CPU: LayerNorm "
                                     "backward (torch autograd dx) with per-sample clipped "
                                     "dgamma/dbeta and noise, median step: bf16 "
                                     f"{res4['bfloat16'][0]:.4f} s over {res4['bfloat16'][1]} "
                                     f"steps, fp32 {res4['float32'][0]:.4f} s over "
                                     f"{res4['float32'][1]} steps (GB/s on the bf16 algorithmic "
                                     "bytes)"}
    finally:
        torch.set_num_threads(prev)
    return out


def cpu_baseline_cfg2():
    """The reference's torch path (flashdp/core/linear_clip.py:94-104 + layers/linear.py:72-80),
    restated in oracle/torch_ref.py, on every core this process may use: the full cfg2
    batch in the config dtype (bf16) and in fp32.  `value` is the bf16 leg."""
    threads, machine = host_cores()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        t16, n16 = _cpu_leg(torch.bfloat16, 12.0)
        t32, n32 = _cpu_leg(torch.float32, 8.0)
    finally:
        torch.set_num_threads(prev)
    F = 2.0 * 8 * 1024 * 3072 * 768
    return {"value": round(F / t16 / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": "cfg2 full batch (B=8,T=1024,768->3072) on CPU, reference torch op sequence "
                      "(per-sample einsum/norm/clamp/mul/sum, /B, normal add), median step "
                      f"after 1 warm-up: bf16 {t16:.4f} s/step over {n16} steps (value), "
                      f"fp32 {t32:.4f} s/step over {n32} steps",
            "fp32_value": round(F / t32 / 1e12, 4),
            "machine_cores": machine,
            "cpu_model": cpu_model()}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the machine type."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


# ------------------------------------------------------------------------ cfg5
def _attention(q, k, v):
    """Causal attention on a fused backend (flash / memory-efficient); the plain
    math backend is excluded because its bf16 batched products with transposed
    operands are avoided on these GPUs.  Falls back to fp32 products."""
    import torch.nn.functional as F
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, is_causal=True)
    except (RuntimeError, ImportError):
        T = q.shape[-2]
        qf, kf, vf = q.float(), k.float().transpose(-1, -2).contiguous(), v.float().contiguous()
        att = torch.matmul(qf, kf) / math.sqrt(q.shape[-1])
        mask = torch.ones(T, T, device=q.device, dtype=torch.bool).tril()
        att = att.masked_fill(~mask, float("-inf")).softmax(-1)
        return torch.matmul(att, vf).to(q.dtype)


def gpt_model(n_layer=24, d=2048, n_head=16, ffn=8192, vocab=50257, ctx=1024):
    """GPT-2-style decoder (pre-LN, no Linear bias, GELU MLP, lm_head tied to the
    token embedding as in the reference's example model, example/gpt2/model.py:111-114),
    random init: 1.313 B parameters at the defaults."""
    import torch.nn as nn
    import torch.nn.functional as F

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln_1 = nn.LayerNorm(d)
            self.c_attn = nn.Linear(d, 3 * d, bias=False)
            self.c_proj = nn.Linear(d, d, bias=False)
            self.ln_2 = nn.LayerNorm(d)
            self.c_fc = nn.Linear(d, ffn, bias=False)
            self.mlp_proj = nn.Linear(ffn, d, bias=False)

        def forward(self, x):
            B, T, C = x.shape
            q, k, v = self.c_attn(self.ln_1(x)).split(C, dim=2)
            q, k, v = (t.view(B, T, n_head, C // n_head).transpose(1, 2) for t in (q, k, v))
            y = _attention(q, k, v).transpose(1, 2).reshape(B, T, C)
            x = x + self.c_proj(y)
            return x + self.mlp_proj(F.gelu(self.c_fc(self.ln_2(x))))

    class GPT(nn.Module):
        def __init__(self):
            super().__init__()
            self.wte = nn.Embedding(vocab, d)
            self.wpe = nn.Embedding(ctx, d)
            self.h = nn.ModuleList(Block() for _ in range(n_layer))
            self.ln_f = nn.LayerNorm(d)
            self.lm_head = nn.Linear(d, vocab, bias=False)
            for m in self.modules():
                if isinstance(m, (nn.Linear, nn.Embedding)):
                    nn.init.normal_(m.weight, std=0.02)
            self.lm_head.weight = self.wte.weight  # weight tying

        def forward(self, idx):
            pos = torch.arange(idx.shape[1], device=idx.device)
            x = self.wte(idx) + self.wpe(pos)
            for blk in self.h:
                x = blk(x)
            return self.lm_head(self.ln_f(x))

    return GPT()


def cfg5_training(dev, steps=10, warmup=3, n_layer=24, fused_adam=True):
    """Tokens/s of full training steps (fwd, bwd, Adam) of the cfg5 decoder, plain and
    with every Linear/LayerNorm except lm_head wrapped by wrap_with_flashdp_layers
    (C=1, sigma=1), bf16 weights, B=8, T=1024, uniform random token ids."""
    import contextlib
    import copy
    import torch.nn as nn
    import torch.nn.functional as F
    from flashdp4review_amd import wrap_with_flashdp_layers
    B, T, V = 8, 1024, 50257
    torch.manual_seed(0)
    with torch.device(dev):
        base = gpt_model(n_layer=n_layer).to(torch.bfloat16)
    n_params = sum(p.numel() for p in base.parameters())  # (the tied head counted once)
    g = torch.Generator(device=dev).manual_seed(0)
    idx = torch.randint(0, V, (B, T + 1), device=dev, generator=g)
    x, y = idx[:, :-1].contiguous(), idx[:, 1:].contiguous()

    def run(model):
        # fused Adam (one multi-tensor kernel per parameter group) where the
        # build has it, else the foreach implementation; the same for both legs
        try:
            opt = torch.optim.Adam(model.parameters(), lr=1e-5, fused=fused_adam,
                                   foreach=None if fused_adam else True)
        except (RuntimeError, ValueError):
            opt = torch.optim.Adam(model.parameters(), lr=1e-5, foreach=True)

        def step():
            logits = model(x)
            loss = F.cross_entropy(logits.view(-1, V).float(), y.view(-1))
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
            return loss

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(steps):
            loss = step()
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / steps
        return ms, float(loss.item())

    ms_plain, loss_plain = run(base)
    dp = copy.deepcopy(base)
    with contextlib.redirect_stdout(sys.stderr):
        wrap_with_flashdp_layers(dp, target_modules=[nn.Linear, nn.LayerNorm],
                                 skip_layers=["lm_head"], C=1.0, noise_multiplier=1.0,
                                 feedback=False)
    del base
    torch.cuda.empty_cache()
    ms_dp, loss_dp = run(dp)
    del dp
    torch.cuda.empty_cache()
    tok = B * T
    return {"workload": f"cfg5: GPT-2-style decoder {n_layer}L d=2048 h=16 ffn=8192 V=50257, "
                        f"tied lm_head, {n_params / 1e9:.3f} B params, B=8 T=1024 bf16, Adam, "
                        "C=1 sigma=1",
            "dp_tokens_per_s": round(tok / ms_dp * 1e3, 1),
            "non_dp_tokens_per_s": round(tok / ms_plain * 1e3, 1),
            "dp_over_non_dp_throughput": round(ms_plain / ms_dp, 4),
            "ms_per_step": {"dp": round(ms_dp, 2), "non_dp": round(ms_plain, 2)},
            "final_loss": {"dp": round(loss_dp, 4), "non_dp": round(loss_plain, 4)},
            "steps": steps, "warmup": warmup}


# ---------------------------------------------------------------------- extras
def weight_and_bias_cost(dev, steps, warmup):
    """cfg2 with a bias: the clipped weight gradient alone and with the bias
    formed in the same launch (fdp_wgrad_bias_clip), each with the default,
    paired kernel and the one-sample wide kernel, and the bias by the separate
    column-sum kernel (what a call without the fused path adds)."""
    from flashdp4review_amd.core import colsum_clip, wgrad_clip
    from flashdp4review_amd.layers.utils import NoiseStream
    x, go, _ = cfg2_inputs(dev)
    B, T, O = go.shape
    keys = NoiseStream()
    bo = torch.empty(O, dtype=torch.bfloat16, device=dev)
    std = 1.0 / math.sqrt(B)

    def w_only():
        wgrad_clip(go, x, 1.0, 1.0, out_scale=1.0 / B, noise_scale=std,
                   noise_key=keys.next(O * x.shape[2]))

    def w_only_one_sample():
        wgrad_clip(go, x, 1.0, 1.0, out_scale=1.0 / B, noise_scale=std,
                   noise_key=keys.next(O * x.shape[2]), single_pass="unpaired")

    def w_and_b(single_pass="auto"):
        wgrad_clip(go, x, 1.0, 1.0, out_scale=1.0 / B, noise_scale=std,
                   noise_key=keys.next(O * x.shape[2]), bias_out=bo, bias_scale=1.0 / (B * T),
                   bias_noise_scale=std, bias_noise_key=keys.next(O), single_pass=single_pass)

    def b_only():
        colsum_clip(go, None, 1.0, 1.0, norm="frob", out_scale=1.0 / (B * T), noise_scale=std,
                    noise_key=keys.next(O))

    tw = median_cuda_time(w_only, steps, warmup, reps=3)
    tw1 = median_cuda_time(w_only_one_sample, steps, warmup, reps=3)
    twb = median_cuda_time(w_and_b, steps, warmup, reps=3)
    twb1 = median_cuda_time(lambda: w_and_b("unpaired"), steps, warmup, reps=3)
    tb = median_cuda_time(b_only, steps, warmup, reps=3)
    return {"weight_ms": round(tw, 4), "weight_one_sample_kernel_ms": round(tw1, 4),
            "weight_and_bias_one_launch_ms": round(twb, 4),
            "weight_and_bias_one_sample_kernel_ms": round(twb1, 4),
            "bias_column_sum_kernel_ms": round(tb, 4),
            "bias_cost_in_launch_us": round((twb - tw) * 1e3, 2),
            "bias_cost_in_one_sample_kernel_us": round((twb1 - tw1) * 1e3, 2)}


def dx_overlap(dev, steps, warmup):
    """DPLinear backward at cfg2: dX = g W (torch's matmul, or the library's own
    dX kernel fdp_dgrad) and the clipped dW/db call, one after the other on one
    stream, or with dX on a second stream (default priority) so that it runs
    beside the DP kernel's tail."""
    from flashdp4review_amd.core import wgrad_clip
    from flashdp4review_amd.layers.utils import NoiseStream
    x, go, _ = cfg2_inputs(dev)
    B, T, O = go.shape
    W = (torch.randn(O, x.shape[2], device=dev) * 0.02).to(torch.bfloat16)
    bo = torch.empty(O, dtype=torch.bfloat16, device=dev)
    keys = NoiseStream()
    std = 1.0 / math.sqrt(B)
    side = torch.cuda.Stream(device=dev)

    def dp():
        wgrad_clip(go, x, 1.0, 1.0, out_scale=1.0 / B, noise_scale=std,
                   noise_key=keys.next(O * x.shape[2]), bias_out=bo, bias_scale=1.0 / (B * T),
                   bias_noise_scale=std, bias_noise_key=keys.next(O))

    def serial():
        go @ W
        dp()

    def overlapped():
        main = torch.cuda.current_stream(dev)
        side.wait_stream(main)
        dp()
        with torch.cuda.stream(side):
            go @ W
        main.wait_stream(side)

    from flashdp4review_amd.core import dgrad

    def serial_own():
        dgrad(go, W, "nn")
        dp()

    t_dx = median_cuda_time(lambda: go @ W, steps, warmup, reps=3)
    t_own = median_cuda_time(lambda: dgrad(go, W, "nn"), steps, warmup, reps=3)
    t_dp = median_cuda_time(dp, steps, warmup, reps=3)
    t_ser = median_cuda_time(serial, steps, warmup, reps=3)
    t_ser_own = median_cuda_time(serial_own, steps, warmup, reps=3)
    t_ovl = median_cuda_time(overlapped, steps, warmup, reps=3)
    return {"dx_gemm_ms": round(t_dx, 4), "dx_fdp_dgrad_ms": round(t_own, 4),
            "dp_weight_bias_ms": round(t_dp, 4), "serial_ms": round(t_ser, 4),
            "serial_with_fdp_dgrad_ms": round(t_ser_own, 4),
            "dx_on_second_stream_ms": round(t_ovl, 4)}


def library_gemms_cfg2(dev, steps, warmup):
    """The same products through hipBLASLt (torch): the non-DP weight gradient
    of the cfg2 layer (one GEMM over all B*T rows, as nn.Linear's backward
    forms it) and the per-sample products materialised by one batched GEMM
    (bmm, no norm, clip or sum).  Both have the clipped kernel's FLOP count."""
    x, go, _ = cfg2_inputs(dev)
    B, T, O = go.shape
    I = x.shape[2]
    g2, x2 = go.reshape(B * T, O), x.reshape(B * T, I)
    gt = go.transpose(1, 2).contiguous()  # [B, O, T]
    F = 2.0 * B * T * I * O
    t_mm = median_cuda_time(lambda: g2.t() @ x2, steps, warmup, reps=3)
    t_bmm = median_cuda_time(lambda: torch.bmm(gt, x), steps, warmup, reps=3)
    return {"non_dp_weight_grad_mm": {"ms": round(t_mm, 4), "tflops": round(F / t_mm / 1e9, 2)},
            "per_sample_bmm_unclipped": {"ms": round(t_bmm, 4),
                                         "tflops": round(F / t_bmm / 1e9, 2)}}


def extra_measurements(dev, steps, warmup):
    import torch.nn as nn
    from flashdp4review_amd import DPLayerNorm, DPLinear
    from flashdp4review_amd.core import layernorm_bwd_clip, layernorm_fwd
    out = {}
    # DP Linear layer fwd+bwd vs nn.Linear (cfg2 shapes, no bias as in GPT-2 MLP)
    x, go, _ = cfg2_inputs(dev)
    lin = nn.Linear(768, 3072, bias=False).to(dev, torch.bfloat16)
    dpl = DPLinear(768, 3072, bias=False, C=1.0, noise_multiplier=1.0).to(dev, torch.bfloat16)
    xr = x.clone().requires_grad_(True)

    def fb(m):
        def f():
            y = m(xr)
            y.backward(go)
        return f

    t_lin = median_cuda_time(fb(lin), steps, warmup, reps=3)
    t_dp = median_cuda_time(fb(dpl), steps, warmup, reps=3)
    out["linear_cfg2_fwd_bwd_ms"] = {"dp": round(t_dp, 4), "non_dp": round(t_lin, 4),
                                     "dp_over_non_dp_throughput": round(t_lin / t_dp, 4)}
    # the same with a bias: DPLinear forms dW and db in one call (fdp_wgrad_bias_clip)
    linb = nn.Linear(768, 3072, bias=True).to(dev, torch.bfloat16)
    dplb = DPLinear(768, 3072, bias=True, C=1.0, noise_multiplier=1.0).to(dev, torch.bfloat16)
    t_linb = median_cuda_time(fb(linb), steps, warmup, reps=3)
    t_dpb = median_cuda_time(fb(dplb), steps, warmup, reps=3)
    out["linear_cfg2_bias_fwd_bwd_ms"] = {"dp": round(t_dpb, 4), "non_dp": round(t_linb, 4),
                                          "dp_over_non_dp_throughput": round(t_linb / t_dpb, 4)}
    out["cfg2_weight_and_bias"] = weight_and_bias_cost(dev, steps, warmup)
    out["cfg2_dx_overlap"] = dx_overlap(dev, steps, warmup)
    # cfg3: Conv1D orientation (x^T g, [768, 2304]) with partially active clipping:
    # the layer's weight and bias gradients in one call (what DPConv1D runs, and
    # what cpu_cfg3 times), the weight alone, and the weight followed by the
    # separate column-sum kernel over grad_output for the bias
    from flashdp4review_amd.core import colsum_clip
    x3, g3 = cfg3_inputs(dev)
    F3 = 2.0 * 16 * 1024 * 768 * 2304
    _, wb3 = run_wgrad(x3, g3, torch.bfloat16, transpose=True, bias=True)
    t3b = median_cuda_time(wb3, steps, warmup, reps=3)
    _, gemm3 = run_wgrad(x3, g3, torch.bfloat16, transpose=True)
    t3 = median_cuda_time(gemm3, steps, warmup, reps=3)

    def two_calls():
        gemm3()
        colsum_clip(g3, None, 1.0, 1.0, norm="frob", out_scale=1.0 / (16 * 1024),
                    noise_scale=0.25, noise_key=(7, 0), out_dtype=torch.bfloat16)
    t3s = median_cuda_time(two_calls, steps, warmup, reps=3)
    from flashdp4review_amd.core import dgrad
    W3 = (torch.randn(768, 2304, device=dev) * 0.02).to(torch.bfloat16)  # Conv1D [nx, nf]
    t3dx = median_cuda_time(lambda: g3 @ W3.t(), steps, warmup, reps=3)
    t3own = median_cuda_time(lambda: dgrad(g3, W3, "nt"), steps, warmup, reps=3)
    out["cfg3_dx"] = {"torch_matmul_ms": round(t3dx, 4), "fdp_dgrad_ms": round(t3own, 4)}
    out["cfg3_conv1d_clipped_wgrad"] = {
        "ms": round(t3b, 4), "tflops": round(F3 / t3b / 1e9, 2),
        "frac_bf16_peak": round(F3 / t3b / 1e9 / PEAK_BF16_TFLOPS, 4),
        "what": "dW and db in one fdp_wgrad_bias_clip call (the bias from the grouped "
                "kernel's grad_output fragments)",
        "weight_only_ms": round(t3, 4),
        "weight_then_column_sum_kernel_ms": round(t3s, 4)}
    # cfg4: LayerNorm H=1024, bf16 I/O, per-sample gamma/beta clip (backward incl. dx)
    g4 = torch.Generator(device=dev).manual_seed(5)
    xl = torch.randn(16, 1024, 1024, device=dev, generator=g4).to(torch.bfloat16)
    gl = (torch.randn(16, 1024, 1024, device=dev, generator=g4) * 0.01).to(torch.bfloat16)
    w = torch.ones(1024, device=dev, dtype=torch.bfloat16)
    _, mean, rstd = layernorm_fwd(xl, w, torch.zeros_like(w), 1e-5)
    tl = median_cuda_time(lambda: layernorm_bwd_clip(gl, xl, w, mean, rstd, 1.0, 1.0), steps,
                          warmup, reps=3)
    nbytes = 3 * 2 * xl.numel() + 8 * 16 * 1024
    out["cfg4_layernorm_bwd_clip"] = {"ms": round(tl, 4), "GBps": round(nbytes / tl / 1e6, 1),
                                      "frac_hbm_peak": round(nbytes / tl / 1e6 / PEAK_HBM_GBS, 4),
                                      "algorithmic_bytes": nbytes}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 200; cfg5: 5)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warm-up steps (default 100, enough for the clocks to settle; "
                         "cfg5: 2)")
    ap.add_argument("--workload", default="cfg2", choices=["cfg2", "cfg3", "cfg4", "cfg5"])
    ap.add_argument("--single-pass", default="auto", choices=["auto", "unpaired", "narrow"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MiB",
                    help="also run one plain device copy of this size (for PMC byte calibration)")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 5 if args.workload == "cfg5" else 200
    if args.warmup is None:
        args.warmup = 2 if args.workload == "cfg5" else 100
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the DP hot path here is single-GPU "
              "(multi-GPU sharding is a design note, not part of this build).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    from flashdp4review_amd import _lib
    _lib.lib()  # fail loudly if the HIP library is missing

    if args.workload == "cfg5":
        r = cfg5_training(dev, steps=args.steps, warmup=args.warmup)
        out = {"metric": "DP-SGD train tokens/s", "value": r["dp_tokens_per_s"],
               "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": r["ms_per_step"]["dp"], "higher_is_better": True,
               "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
               "data": "synthetic (uniform random token ids, random-init weights)",
               "config": {"workload": r["workload"]}, "extra": r,
               "device": torch.cuda.get_device_name(dev)}
        print(json.dumps(out), flush=True)
        return

    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if args.workload == "cfg2":
        x, go, _ = cfg2_inputs(dev)
        B, T, I, O = 8, 1024, 768, 3072
        step, _ = run_wgrad(x, go, torch.bfloat16, single_pass=args.single_pass)
        step_coop, _ = run_wgrad(x, go, torch.bfloat16, launch="cooperative",
                                 single_pass=args.single_pass)
        workload = ("cfg2: DP Linear 768->3072 clipped per-sample weight grad, B=8 T=1024, "
                    "C=1, sigma=1")
    elif args.workload == "cfg3":
        x, go = cfg3_inputs(dev)
        B, T, I, O = 16, 1024, 768, 2304
        step, _ = run_wgrad(x, go, torch.bfloat16, transpose=True, bias=True,
                            single_pass=args.single_pass)
        step_coop, _ = run_wgrad(x, go, torch.bfloat16, transpose=True, launch="cooperative",
                                 bias=True, single_pass=args.single_pass)
        workload = ("cfg3: DP Conv1D 768->2304 clipped per-sample weight and bias grads in one "
                    "call, B=16 T=1024, norms 0.1C..10C")
    else:
        from flashdp4review_amd.core import layernorm_bwd_clip, layernorm_fwd
        g4 = torch.Generator(device=dev).manual_seed(5)
        xl = torch.randn(16, 1024, 1024, device=dev, generator=g4).to(torch.bfloat16)
        gl = (torch.randn(16, 1024, 1024, device=dev, generator=g4) * 0.01).to(torch.bfloat16)
        w = torch.ones(1024, device=dev, dtype=torch.bfloat16)
        _, mean, rstd = layernorm_fwd(xl, w, torch.zeros_like(w), 1e-5)

        from flashdp4review_amd.layers.utils import NoiseStream
        keys = NoiseStream()

        def step():
            return layernorm_bwd_clip(gl, xl, w, mean, rstd, 1.0, 1.0, out_scale=1.0 / 16,
                                      noise_scale=0.25, noise_key=keys.next(1024))

        step_coop = None

    # ---- timed region: K steps bracketed by synchronisation and a pair of HIP
    # events on the launch stream.  A step is one call, and the call is one
    # launch of the dominant kernel (cfg2/cfg3; cfg4: the call's kernels), so
    # the region's mean is that kernel's mean launch duration as well (the
    # roofline's avg_ms; the host issues calls faster than the device runs them,
    # see host_us_per_call).  profiles/ holds the rocprofv3 kernel-trace of
    # the same command, whose average agrees.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        step()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    call_ms = ms
    # host time per call: calls issued back to back while the device is busy
    n_host = 100
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_host):
        step()
    host_us = (time.perf_counter() - t0) / n_host * 1e6
    torch.cuda.synchronize()

    if args.workload == "cfg4":
        # algorithmic bytes: read x, dy, write dx (bf16) + mean/rstd (fp32)
        nbytes = 3 * 2 * 16 * 1024 * 1024 + 8 * 16 * 1024
        res = {"metric": "DP LayerNorm per-sample grad GB/s", "value": round(nbytes / ms / 1e6, 1),
               "unit": "GB/s", "dtype": "bf16",
               "config": {"workload": "cfg4: DP LayerNorm H=1024 bwd incl. dx, B=16 T=1024, "
                                      "per-sample gamma/beta clip, 1/B, noise"}}
        roof = {"bound": "hbm", "achieved": round(nbytes / call_ms / 1e6, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(nbytes / call_ms / 1e6 / PEAK_HBM_GBS, 4),
                "traffic": TRAFFIC_BYTES[("cfg4", "auto")],
                "kernel": "ln_bwd_fused_kernel: one launch per fdp_layernorm_bwd_clip call, "
                          "HIP events around the timed region",
                "bytes_per_launch": nbytes, "avg_ms": round(call_ms, 4)}
    else:
        F = 2.0 * B * T * I * O
        res = {"metric": "clipped per-sample-grad GEMM TFLOP/s", "value": round(F / ms / 1e9, 2),
               "unit": "TFLOP/s", "dtype": "bf16", "config": {"workload": workload}}
        roof = {"bound": "mfma", "achieved": round(F / call_ms / 1e9, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(F / call_ms / 1e9 / PEAK_BF16_TFLOPS, 4),
                "traffic": TRAFFIC_BYTES.get((args.workload, args.single_pass)),
                "kernel": KERNELS.get((args.workload, args.single_pass), "single-pass kernel")
                          + ": one launch per fdp_wgrad_clip call, HIP events around the timed "
                            "region",
                "flops_per_launch": F, "avg_ms": round(call_ms, 4)}
    out = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": res["dtype"], "data": "synthetic (seeded randn, inputs resident in HBM)",
           "config": res["config"], "roofline": roof, "host_us_per_call": round(host_us, 1)}
    if not args.no_cpu_baseline and args.workload == "cfg2":
        out["cpu_baseline"] = cpu_baseline_cfg2()
    if not args.no_extra and args.workload == "cfg2":
        extra = {}
        t_coop = median_cuda_time(step_coop, args.steps, 3, reps=3)
        F = 2.0 * B * T * I * O
        extra["cfg2_step_cooperative_launch"] = {"ms": round(t_coop, 4),
                                                 "tflops": round(F / t_coop / 1e9, 2)}
        step_one, _ = run_wgrad(x, go, torch.bfloat16, single_pass="unpaired")
        t_one = median_cuda_time(step_one, args.steps, 3, reps=3)
        extra["cfg2_step_one_sample_per_cu"] = {"ms": round(t_one, 4),
                                                "tflops": round(F / t_one / 1e9, 2)}
        step_narrow, _ = run_wgrad(x, go, torch.bfloat16, single_pass="narrow")
        t_nar = median_cuda_time(step_narrow, args.steps, 3, reps=3)
        extra["cfg2_step_grouped_kernel"] = {"ms": round(t_nar, 4),
                                             "tflops": round(F / t_nar / 1e9, 2)}
        extra["cfg2_library_gemms"] = library_gemms_cfg2(dev, max(5, args.steps // 5), 3)
        extra.update(extra_measurements(dev, max(5, args.steps // 5), 3))
        extra["cfg5_training"] = cfg5_training(dev)
        if not args.no_cpu_baseline:
            extra.update(cpu_baselines_cfg3_cfg4())
        out["extra"] = extra
    out["device"] = torch.cuda.get_device_name(dev)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
