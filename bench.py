"""Benchmark of the quantized DiT linear path on one MI355X.

Headline (one "step"): the DiT-block linear stack at M = 32768 tokens, hidden 3072 -- QKV 3072->9216,
attention-out 3072->3072, FFN-up 3072->12288, FFN-down 12288->3072 -- as W8A8 int8 GEMMs with per-token
int8 activations (already quantized and resident in HBM), per-channel int8 weights, bf16 bias and bf16
outputs.  value = 2*M*N*K summed over the four GEMMs / step time, in TOPS (10^12 int8 ops/s).

The same JSON line carries:
  roofline      the GEMM kernel's achieved TOPS from per-launch HIP events vs the dense int8 MFMA peak;
  cpu_baseline  the reference's CPU fallback (dequantize the weight, bf16 F.linear) on a bounded row sample
                of the same four GEMMs, timed on this host;
  extra         the stack with activation quantization included, the reference's g128 scale layout,
                the block-scaled fp8 GEMMs, and the fused elementwise kernels' HBM bandwidth.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-extra] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "comfyui-hy-nomas_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

M = 32768
HIDDEN = 3072
# Memory-side bytes per headline step (4 GEMM launches) from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this
# script, scaled by a plain-copy calibration (FETCH x2.0, WRITE x1.0); profiles/block_gemm_int8_per_token_M32768.md
TRAFFIC_BYTES_PER_STEP = 6.56e9
SLEEP_CYCLES = 2e8           # ~80 ms of spin before each timed region
HOT_S = 0.1                  # seconds of untimed passes between the spin and the timed region
HOT_MAX_LAUNCHES = 2000
WARM_S = 1.5                 # seconds of untimed GEMM work before the headline's timed region
STACK = [("qkv", 3072, 9216), ("attn_out", 3072, 3072), ("ffn_up", 3072, 12288), ("ffn_down", 12288, 3072)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def outlier_activations(m, k, gen, dev):
    """bf16 ~N(0, 1) with 1% of the channels scaled x20."""
    x = torch.randn(m, k, generator=gen, device=dev)
    ch = torch.randperm(k, generator=gen, device=dev)[: k // 100]
    x[:, ch] *= 20
    return x.to(torch.bfloat16)


def make_linear(n, k, gen, dev, groups):
    w = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
    sw = torch.rand(n, groups, generator=gen, device=dev) * 4e-3 + 1e-3
    bias = (torch.randn(n, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    return w, sw.float(), bias


def time_launches(fns, steps, warmup, warm_s=0.0):
    """Run the list of launches `steps` times; returns (ms per step, [avg ms per launch]) from HIP events
    recorded on the current stream (the stream the kernels are launched on): the step time from one event
    pair around all steps, the per-launch averages from a second pass with an event pair around every launch.
    Before the timed region: `warmup` untimed passes, then more untimed passes until `warm_s` seconds have
    elapsed, so the GPU clocks reach the steady state of this work (they take about a second to settle under
    a matrix-core load).

    Each timed pass is queued behind a spin kernel, so the events measure GPU time and not the host's
    per-call overhead (which exceeds a 50 us elementwise kernel).  The spin leaves the chip nearly idle for
    ~80 ms, and the first ~30 ms of matrix-core work after such an idle period run up to 25 % slower than
    the sustained rate while the power controller settles; so HOT_S seconds of untimed passes sit between
    the spin and the start event."""
    for _ in range(warmup):
        for f in fns:
            f()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    passes = 0
    while passes == 0 or time.perf_counter() - t0 < warm_s:
        for f in fns:
            f()
        torch.cuda.synchronize()
        passes += 1
    pass_s = (time.perf_counter() - t0) / passes
    hot = max(1, min(int(HOT_S / pass_s) + 1, HOT_MAX_LAUNCHES // len(fns)))
    stream = torch.cuda.current_stream()
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in fns]
          for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spin0 = torch.cuda.Event(enable_timing=True)

    def spin_then_hot():
        torch.cuda.synchronize()
        t = time.perf_counter()
        spin0.record(stream)
        torch.cuda._sleep(int(SLEEP_CYCLES))
        for _ in range(hot):
            for f in fns:
                f()
        return t

    t = spin_then_hot()
    start.record(stream)
    for s in range(steps):
        for f in fns:
            f()
    end.record(stream)
    host_s = time.perf_counter() - t
    torch.cuda.synchronize()
    ahead_ms = spin0.elapsed_time(start)
    if host_s * 1e3 > ahead_ms:
        log(f"bench: host queueing took {host_s * 1e3:.1f} ms, the GPU reached the timed region after "
            f"{ahead_ms:.1f} ms: part of the timed region waited for the host")
    total_ms = start.elapsed_time(end) / steps
    # a second pass with an event pair around every launch, for the per-launch averages
    spin_then_hot()
    for s in range(steps):
        for i, f in enumerate(fns):
            ev[s][i][0].record(stream)
            f()
            ev[s][i][1].record(stream)
    torch.cuda.synchronize()
    per = [sum(ev[s][i][0].elapsed_time(ev[s][i][1]) for s in range(steps)) / steps for i in range(len(fns))]
    return total_ms, per


def gemm_stack(dev, gen, steps, warmup, group_mode="per_token", kind="int8", warm_s=WARM_S, expand=False):
    """Headline stack.  Returns (ms/step, per-GEMM ms, total ops, [(name, K, N)])."""
    from hy_nomas import kernels

    fns, ops, keep = [], 0, []
    for name, k, n in STACK:
        x = outlier_activations(M, k, gen, dev)
        if kind == "int8":
            groups = 1 if group_mode == "per_token" else k // 128
            qa, sa = kernels.quantize_activations(x, "int8", None if group_mode == "per_token" else 128)
            w, sw, bias = make_linear(n, k, gen, dev, groups)
        else:
            from hy_nomas import pixelumm
            qa, sa = kernels.quantize_activations(x, "fp8", 128)
            wf = torch.randn(n, k, generator=gen, device=dev) * 0.02
            w, sblk = pixelumm.quantize_fp8_block(wf)
            # [N/128, K/128] block scales, read directly by the GEMM; expand: one row per output channel,
            # as the reference hands them to its kernel (pixelumm.py:153, repeat_interleave(128, 0))
            sw = sblk.repeat_interleave(128, 0)[:n].contiguous() if expand else sblk
            bias = (torch.randn(n, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            del wf
        del x
        keep.append((qa, sa, w, sw, bias))
        fns.append(lambda qa=qa, sa=sa, w=w, sw=sw, bias=bias: kernels.block_gemm(qa, sa, w, sw, bias, kind=kind))
        ops += 2 * M * n * k
    ms, per = time_launches(fns, steps, warmup, warm_s)
    del keep, fns
    torch.cuda.empty_cache()
    return ms, per, ops


def linear_stack_with_quant(dev, gen, steps, warmup):
    """The four linears from bf16 activations: per-token quantization + GEMM each (block_linear)."""
    from hy_nomas import kernels

    fns, keep = [], []
    for name, k, n in STACK:
        x = outlier_activations(M, k, gen, dev)
        w, sw, bias = make_linear(n, k, gen, dev, 1)
        keep.append((x, w, sw, bias))
        fns.append(lambda x=x, w=w, sw=sw, bias=bias: kernels.block_linear(x, w, sw, bias))
    ms, _ = time_launches(fns, steps, warmup)
    del keep, fns
    torch.cuda.empty_cache()
    return ms


def decoder_mlp(dev, gen, steps, warmup):
    """PixelUMM decoder MLP on fp8 block weights at the reference's kernel-bench shape (M=35200 tokens,
    hidden 4096, intermediate 12288): down(silu(gate(x)) * up(x)).  "fused": x quantized once, gate and up
    in one GEMM whose epilogue writes the e4m3 codes of the SwiGLU product, then the down GEMM.
    "unfused": the reference's order (three fp8 linears, torch's bf16 silu and product)."""
    from hy_nomas import kernels, pixelumm

    m, hid, inter = 35200, 4096, 12288
    x = outlier_activations(m, hid, gen, dev)
    ws = {}
    for name, (o, k) in {"gate": (inter, hid), "up": (inter, hid), "down": (hid, inter)}.items():
        ws[name] = pixelumm.quantize_fp8_block(torch.randn(o, k, generator=gen, device=dev) * 0.02)
    gate_up = pixelumm.interleave_gate_up(ws["gate"], ws["up"])
    fused = [lambda: pixelumm.swiglu_mlp(x, gate_up, ws["down"])]
    lin = pixelumm.fp8_block_linear
    unfused = [lambda: lin(torch.nn.functional.silu(lin(x, *ws["gate"])) * lin(x, *ws["up"]), *ws["down"])]
    ops = 2 * m * hid * inter * 3
    out = {"M": m, "hidden": hid, "intermediate": inter}
    for name, fns in (("fused", fused), ("unfused", unfused)):
        ms, _ = time_launches(fns, steps, warmup, WARM_S)
        out[name] = {"ms": round(ms, 4), "TFLOPS": round(ops / (ms * 1e-3) / 1e12, 1)}
    # the fused path's two GEMMs alone, per launch
    qa, sa = kernels.quantize_activations(x, "fp8")
    hq, hs = kernels.block_gemm(qa, sa, *gate_up, kind="fp8", epilogue="swiglu_quant")
    _, per = time_launches([lambda: kernels.block_gemm(qa, sa, *gate_up, kind="fp8", epilogue="swiglu_quant"),
                            lambda: kernels.block_gemm(hq, hs, *ws["down"], kind="fp8")], steps, warmup)
    out["gate_up_swiglu_gemm"] = {"ms": round(per[0], 4), "TFLOPS": round(2 * m * hid * 2 * inter / (per[0] * 1e-3) / 1e12, 1)}
    out["down_gemm"] = {"ms": round(per[1], 4), "TFLOPS": round(2 * m * inter * hid / (per[1] * 1e-3) / 1e12, 1)}
    del x, ws, gate_up, qa, sa, hq, hs, fused, unfused
    torch.cuda.empty_cache()
    return out


def modulation_linear(dev, gen, steps, warmup):
    """The per-sample modulation linear of a double-stream block (hy_nomas/model.py:306-314): silu(vec)
    [B, 3072] -> [B, 18432] with Tencent's int8 g128 weight, at B = 1 and 2: the skinny int8 kernel,
    bound by the 56.6 MB weight stream.  Eight weight copies rotate (453 MB > the Infinity Cache)."""
    from hy_nomas import kernels

    k, n = HIDDEN, 6 * HIDDEN
    ws = []
    for _ in range(8):
        w = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
        sw = torch.rand(n, k // 128, generator=gen, device=dev) * 4e-3 + 1e-3
        ws.append((w, sw.float(), (torch.randn(n, generator=gen, device=dev) * 0.02).to(torch.bfloat16)))
    nbytes = n * k + n * (k // 128) * 4
    out = {"N": n, "K": k, "weight_bytes": nbytes}
    for b in (1, 2):
        qa, sa = kernels.quantize_activations(torch.randn(b, k, generator=gen, device=dev).to(torch.bfloat16))
        fns = [lambda w=w: kernels.block_gemm(qa, sa, w[0], w[1], w[2]) for w in ws]
        total_ms, _ = time_launches(fns, steps, warmup)
        us = 1e3 * total_ms / len(fns)
        out[f"B{b}"] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1),
                        "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 3)}
    del ws
    torch.cuda.empty_cache()
    return out


def kv_history(dev, gen, steps, warmup):
    """int8 K/V history of the config-4 block: K [57344, 24, 128] bf16, quantized per (token, head) and
    dequantized back to bf16, two rotating slabs (> the 256 MB Infinity Cache together with their codes)."""
    from hy_nomas import kv

    shape = (57344, 24, 128)
    n_el = shape[0] * shape[1] * shape[2]
    xs = [torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
    qs = [kv.quantize_kv(x) for x in xs]
    out = {}
    for name, fns, nbytes in (
            ("quantize_kv", [lambda x=x: kv.quantize_kv(x) for x in xs], n_el * (2 + 1) + n_el // 128 * 4),
            ("dequantize_kv", [lambda q=q: kv.dequantize_kv(q[0], q[1]) for q in qs], n_el * (1 + 2) + n_el // 128 * 4)):
        total_ms, per = time_launches(fns, steps, warmup)
        us = 1e3 * total_ms / len(fns)
        out[name] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1),
                     "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 3), "bytes": int(nbytes)}
    del xs, qs
    torch.cuda.empty_cache()
    return out


def elementwise(dev, gen, steps, warmup):
    """Fused elementwise kernels at x [1, 32768, 3072] bf16, three rotating input sets (576 MiB > the 256 MB
    Infinity Cache) so each launch reads cold HBM.  Returns {name: (us, GB/s, algorithmic bytes)}."""
    from hy_nomas import fused, kernels

    n_el = M * HIDDEN
    sets = []
    for _ in range(3):
        x = torch.randn(1, M, HIDDEN, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.randn(1, M, HIDDEN, generator=gen, device=dev).to(torch.bfloat16)
        sets.append((x, y))
    shift = (torch.randn(1, HIDDEN, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
    scale = (torch.randn(1, HIDDEN, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
    gate = (torch.randn(1, HIDDEN, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
    # camera output per latent frame: 32 frames of 1024 tokens
    frames = (torch.randn(1, 32, HIDDEN, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
    # QK norms: 24 heads x 128, per-token rotary tables [M, 128] fp32 (read by every head of the token)
    heads, hd = HIDDEN // 128, 128
    qn_w = (torch.rand(hd, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
    ang = torch.rand(M, hd, generator=gen, device=dev) * 6.283
    cos_t, sin_t = torch.cos(ang), torch.sin(ang)
    wt = (torch.rand(hd // 2, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
    whw = (torch.rand(hd // 2, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
    tables_bpe = 2.0 * M * hd * 4 / n_el
    cases = {
        "adaln": (lambda s: fused.adaln(s[0], shift, scale), 4.0),
        "gated_residual": (lambda s: fused.gated_residual(s[0], s[1], gate), 6.0),
        "gated_residual_frames": (lambda s: fused.gated_residual_frames(s[0], s[1], gate, frames), 6.0),
        "adaln_quant": (lambda s: kernels.adaln_quant(s[0], shift, scale), 3.0 + 4.0 / 128),
        "adaln_quant_per_token": (lambda s: kernels.adaln_quant(s[0], shift, scale, group=None), 3.0 + 4.0 / HIDDEN),
        "quantize_g128": (lambda s: kernels.quantize_activations(s[0].view(M, HIDDEN)), 3.0 + 4.0 / 128),
        "quantize_per_token": (lambda s: kernels.quantize_activations(s[0].view(M, HIDDEN), "int8", None),
                               3.0 + 4.0 / HIDDEN),
        "qk_norm_rope": (lambda s: fused.qk_norm_rope(s[0].view(1, M, heads, hd), qn_w, (cos_t, sin_t)),
                         4.0 + tables_bpe),
        "pixelumm_qk": (lambda s: fused.pixelumm_qk(s[0].view(1, M, heads, hd), wt, whw, cos_t, sin_t),
                        4.0 + tables_bpe),
    }
    out = {}
    for name, (fn, bpe) in cases.items():
        fns = [lambda s=s, fn=fn: fn(s) for s in sets]
        total_ms, per = time_launches(fns, steps, warmup)
        # us: back-to-back launches on one stream (the kernel's throughput, launch gaps included);
        # us_event: an event pair around each launch (adds the event overhead)
        us = 1e3 * total_ms / len(fns)
        nbytes = bpe * n_el
        out[name] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1),
                     "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 3), "bytes": int(nbytes),
                     "us_event": round(1e3 * sum(per) / len(per), 2)}
    del sets
    torch.cuda.empty_cache()
    return out


def rope_tables(length, head_dim, gen, dev):
    """cos / sin [length, head_dim] fp32 of random angles, each repeated for its interleaved pair (the shape
    and layout of the model's 3-D RoPE tables; the values do not change the work)."""
    ang = torch.rand(length, head_dim // 2, generator=gen, device=dev) * 6.283
    return ang.cos().repeat_interleave(2, dim=1), ang.sin().repeat_interleave(2, dim=1)


def dit_block(dev, gen, steps, warmup, per_token):
    """One synthetic double-stream DiT block forward (hy_nomas/model.py:230-286) at hidden 3072, 24 heads x 128,
    FFN 12288 GELU-tanh: 57344 image tokens (RoPE grid 14 x 64 x 64) + 256 text tokens, random int8 weights,
    joint attention with torch SDPA (the default) and with the HIP attention kernel.  For each backend:
    {"block_ms", "attention_ms", "linear_path_ms", "linear_TOPS"}; the linear path (every other kernel of this
    package) is the block time minus the attention time of the same shapes, timed as the block calls it."""
    from hy_nomas import attention, block

    d, heads, mlp, lv, lt = HIDDEN, 24, 12288, 57344, 256

    def linear(n, k):
        qw = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
        sw = torch.rand(n, 1 if per_token else k // 128, generator=gen, device=dev) * 2e-3 + 5e-4
        bias = (torch.randn(n, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        return block.Int8Linear(qw, sw.float(), bias)

    def stream():
        lins = [linear(n, k) for n, k in ((3 * d, d), (d, d), (mlp, d), (d, mlp))]
        qn = (torch.rand(d // heads, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
        kn = (torch.rand(d // heads, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
        return block.DiTBlockInt8(*lins, qn, kn, heads, per_token=per_token)

    blk = block.DoubleStreamBlockInt8(stream(), stream())
    img = torch.randn(1, lv, d, generator=gen, device=dev).to(torch.bfloat16)
    txt = torch.randn(1, lt, d, generator=gen, device=dev).to(torch.bfloat16)
    mods = [[(torch.randn(1, d, generator=gen, device=dev) * 0.1).to(torch.bfloat16) for _ in range(6)]
            for _ in range(2)]
    rope = rope_tables(lv, d // heads, gen, dev)
    out = {"activations": "per-token x per-channel" if per_token else "g128 (reference layout)"}
    ops = 2 * (lv + lt) * sum(n * k for _, k, n in STACK)
    # the block's attention call on the same operands: head-major q, k, v [B, H, L, D] as the QKV epilogue
    # writes them, image and text tokens together (SDPA); for the HIP kernel, q and k head-major and v in the
    # V^T layout the QKV epilogue writes for it
    hm = torch.randn(3, 1, heads, lv + lt, d // heads, generator=gen, device=dev).to(torch.bfloat16)
    vt = attention.transpose_values(hm[2])
    att_flops = 4 * (lv + lt) ** 2 * d
    att_calls = {"sdpa": lambda: attention.attention_heads(hm[0], hm[1], hm[2], "sdpa"),
                 "hip": lambda: attention.attention_hip(hm[0].transpose(1, 2), hm[1].transpose(1, 2), vt, lv + lt)}
    with torch.no_grad():
        for backend in ("sdpa", "hip"):
            ms, _ = time_launches([lambda: blk.forward(img, txt, mods[0], mods[1], rope, backend)], steps, warmup)
            att_ms, _ = time_launches([att_calls[backend]], steps, warmup)
            lin_ms = ms - att_ms
            out[backend] = {"block_ms": round(ms, 3), "attention_ms": round(att_ms, 3),
                            "attention_TFLOPS": round(att_flops / (att_ms * 1e-3) / 1e12, 1),
                            "linear_path_ms": round(lin_ms, 3), "linear_TOPS": round(ops / (lin_ms * 1e-3) / 1e12, 1)}
    del blk, img, txt, hm, vt
    torch.cuda.empty_cache()
    out["linear_ops"] = ops
    out["attention_flops"] = att_flops
    return out


def attention_only(dev, gen, steps, warmup):
    """The block's joint attention alone at 57344 + 256 tokens x 24 heads x 128, on the operands the block's QKV
    epilogue writes for each backend: head-major bf16 q, k, v for SDPA; q and k head-major and v as V^T for the
    HIP kernel.  ms and TFLOPS (4 L^2 D H flops); "hip_with_vt_copy" adds the V^T copy a caller with head-major
    v makes (`attention.attention_heads`)."""
    from hy_nomas import attention

    length, heads = 57344 + 256, 24
    hm = torch.randn(3, 1, heads, length, 128, generator=gen, device=dev).to(torch.bfloat16)
    vt = attention.transpose_values(hm[2])
    flops = 4 * length ** 2 * 128 * heads
    out = {"tokens": length, "heads": heads, "flops": flops}
    calls = {"sdpa": lambda: attention.attention_heads(hm[0], hm[1], hm[2], "sdpa"),
             "hip": lambda: attention.attention_hip(hm[0].transpose(1, 2), hm[1].transpose(1, 2), vt, length),
             "hip_with_vt_copy": lambda: attention.attention_heads(hm[0], hm[1], hm[2], "hip")}
    with torch.no_grad():
        for name, fn in calls.items():
            ms, _ = time_launches([fn], steps, warmup)
            out[name] = {"ms": round(ms, 3), "TFLOPS": round(flops / (ms * 1e-3) / 1e12, 1)}
    del hm, vt
    torch.cuda.empty_cache()
    return out


# the linears of the reference's own kernel benchmark (dev/bench_kernels.py:27-28): the released checkpoint's
# hidden 2048 / FFN 8192 DiT at 26400 tokens, the PixelUMM decoder's 4096 <-> 12288 MLP at 35200, and an M=300
# text-length case; weights N(0, 0.02) in Tencent's g128 int8 layout, activations N(0, 2)
REF_SHAPES = [(26400, 2048, 2048), (26400, 2048, 8192), (26400, 8192, 2048), (35200, 4096, 12288),
              (35200, 12288, 4096), (300, 2048, 12288)]


def reference_shapes(dev, gen, steps, warmup):
    """Per launch at each of the reference benchmark's shapes: our int8_g128_linear (g128 activation
    quantization + GEMM, the reference's call), the GEMM alone on pre-quantized activations, the fp8 block
    linear (block scales read as stored, and expanded per channel as the reference passes them), and
    torch's bf16 F.linear on the dequantized weight (hipBLASLt), with the relative error of the int8 path
    against that bf16 product (the reference script's figure)."""
    from hy_nomas import kernels, ops, pixelumm

    F = torch.nn.functional
    rows = []
    for m, k, n in REF_SHAPES:
        x = (torch.randn(m, k, generator=gen, device=dev) * 2).to(torch.bfloat16)
        w = torch.randn(n, k, generator=gen, device=dev) * 0.02
        bias = torch.randn(n, generator=gen, device=dev).to(torch.bfloat16)
        q, sc = ops.quantize_g128(w)
        wd = ops.dequantize_g128(q, sc)
        qf, sf = pixelumm.quantize_fp8_block(w)
        sfx = sf.repeat_interleave(128, 0).contiguous()
        del w
        ref = F.linear(x, wd, bias).float()
        err = ((kernels.int8_g128_linear(x, q, sc, bias).float() - ref).norm() / ref.norm()).item()
        err8 = ((pixelumm.fp8_block_linear(x, qf, sf, bias).float() - ref).norm() / ref.norm()).item()
        del ref
        qa, sa = kernels.quantize_activations(x)
        fns = [lambda: kernels.int8_g128_linear(x, q, sc, bias),
               lambda: kernels.block_gemm(qa, sa, q, sc, bias),
               lambda: pixelumm.fp8_block_linear(x, qf, sf, bias),
               lambda: kernels.block_linear(x, qf, sfx, bias, kind="fp8"),
               lambda: F.linear(x, wd, bias)]
        _, per = time_launches(fns, steps, warmup, 0.3)
        ops_ = 2 * m * n * k
        row = {"M": m, "K": k, "N": n, "int8_rel_err_vs_bf16": float(f"{err:.3e}"),
               "fp8_rel_err_vs_bf16": float(f"{err8:.3e}")}
        for name, t, peak in (("int8_g128_linear", per[0], PEAK_INT8_TOPS), ("int8_g128_gemm", per[1], PEAK_INT8_TOPS),
                              ("fp8_block_linear", per[2], PEAK_FP8_TFLOPS),
                              ("fp8_linear_expanded_scales", per[3], PEAK_FP8_TFLOPS),
                              ("bf16_F_linear_hipblaslt", per[4], 2500.0)):
            tops = ops_ / (t * 1e-3) / 1e12
            row[name] = {"ms": round(t, 4), "TOPS": round(tops, 1), "frac_peak": round(tops / peak, 3)}
        rows.append(row)
        del x, q, sc, wd, qf, sf, sfx, qa, sa, bias, fns
        torch.cuda.empty_cache()
    return rows


def peaks(dev, gen):
    """The roofline denominators measured on this GPU with the committed probes (csrc/probes/peak.hip):
    int8 and fp8 MFMA loops on real operand data (activation-like codes x weight codes; the power limit,
    and with it the clock, depends on the data), two waves per SIMD, with the shader clock they ran at; and
    a streaming 1 GiB device copy.  The roofline fraction stays against the published peaks; these show
    what the chip sustains."""
    import ctypes

    from hy_nomas import kernels, pixelumm

    path = os.path.join(ROOT, "comfyui-hy-nomas_amd", "hy_nomas", "libhynomas_probes.so")
    lib = ctypes.CDLL(path)
    i64, vp, ci = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    lib.hnp_operand_bytes.restype, lib.hnp_operand_bytes.argtypes = i64, [ci]
    lib.hnp_ops_per_mfma.restype, lib.hnp_ops_per_mfma.argtypes = i64, [ci]
    lib.hnp_mfma_loop.argtypes = [ci, vp, vp, ci, ci, vp, vp, vp]
    lib.hnp_copy.argtypes = [vp, vp, i64, ci, vp]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks = 2 * cus                      # 8 waves per CU, two per SIMD (as the GEMM runs)
    waves = blocks * lib.hnp_waves_per_block()
    stream = torch.cuda.current_stream()
    out = {"compute_units": cus}
    for kind, name, peak in ((0, "int8_mfma", PEAK_INT8_TOPS), (1, "fp8_mfma", PEAK_FP8_TFLOPS)):
        nbytes = lib.hnp_operand_bytes(kind)
        x = outlier_activations(nbytes // 256, 256, gen, dev)
        if kind == 0:
            a, _ = kernels.quantize_activations(x, "int8", None)
            b = torch.randint(-127, 128, (nbytes,), generator=gen, device=dev, dtype=torch.int8)
        else:
            a, _ = kernels.quantize_activations(x, "fp8", 128)
            b, _ = pixelumm.quantize_fp8_block(torch.randn(nbytes // 256, 256, generator=gen, device=dev) * 0.02)
        a, b = a.contiguous(), b.contiguous()
        res = torch.empty(waves * 64, dtype=torch.int32, device=dev)
        clk = torch.zeros(2, dtype=torch.int64, device=dev)
        iters = 20000

        def launch():
            rc = lib.hnp_mfma_loop(kind, a.data_ptr(), b.data_ptr(), iters, blocks, res.data_ptr(), clk.data_ptr(),
                                   stream.cuda_stream)
            if rc:
                raise RuntimeError(f"hnp_mfma_loop failed ({rc})")

        t0 = time.perf_counter()
        while time.perf_counter() - t0 < WARM_S:
            launch()
            torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(stream)
        for _ in range(5):
            launch()
        ev[1].record(stream)
        torch.cuda.synchronize()
        ms = ev[0].elapsed_time(ev[1]) / 5
        ops = waves * iters * lib.hnp_mfma_per_iter() * lib.hnp_ops_per_mfma(kind)
        cycles, ticks = clk.tolist()
        tops = ops / (ms * 1e-3) / 1e12
        out[name] = {"TOPS": round(tops, 1), "frac_published_peak": round(tops / peak, 3),
                     "clock_GHz": round(cycles / (ticks / 100e6) / 1e9, 3), "ms_per_launch": round(ms, 3)}
        del a, b, x, res, clk
    nb = 1 << 30
    src = torch.empty(nb, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(7)

    def copy():
        if lib.hnp_copy(src.data_ptr(), dst.data_ptr(), nb, cus * 8, stream.cuda_stream):
            raise RuntimeError("hnp_copy failed")

    for _ in range(3):
        copy()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record(stream)
    for _ in range(10):
        copy()
    ev[1].record(stream)
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / 10
    gbs = 2 * nb / (ms * 1e-3) / 1e9
    out["copy_1GiB"] = {"GB/s": round(gbs, 1), "frac_published_peak": round(gbs / PEAK_HBM_GBS, 3),
                        "ms": round(ms, 3)}
    del src, dst
    torch.cuda.empty_cache()
    return out


def config0_gpu(dev, steps, warmup):
    """The CPU-baseline workload on the GPU: x bf16 [1024, 3072] ~N(0, 1) with 1 % of the channels x20,
    per-token int8 quantization with round-half-even, per-channel int8 weights [3072, 3072] with fp32 scales
    ~U(1e-3, 5e-3), bf16 bias, bf16 out; seed 0.  Quantization + GEMM per launch."""
    from hy_nomas import kernels

    m, k, n = 1024, HIDDEN, HIDDEN
    g = torch.Generator().manual_seed(0)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[: k // 100]] *= 20
    x = x.to(torch.bfloat16).to(dev)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
    sw = (torch.rand(n, 1, generator=g) * 4e-3 + 1e-3).to(dev)
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).to(dev)

    def linear():
        qa, sa = kernels.quantize_activations(x, "int8", None, rounding="half_even")
        return kernels.block_gemm(qa, sa, w, sw, bias)

    _, per = time_launches([linear], steps, warmup, 0.3)
    ops = 2 * m * n * k
    return {"ms": round(per[0], 4), "TOPS": round(ops / (per[0] * 1e-3) / 1e12, 1), "ops": ops,
            "workload": "W8A8 linear 1024x3072 -> 3072, per-token half-even int8 activations, per-channel "
                        "int8 weights, bias, bf16 out (quantization + GEMM)"}


def cpu_host():
    """The host CPU: model name, logical CPUs, CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity}


# Threads for the CPU legs: a one-GPU job on the MI355X hosts this runs on has a 16-CPU share (its worker
# pools and OMP_NUM_THREADS are sized to it), whatever the host's CPU count.
CPU_SHARE = 16


def cpu_baseline(target_s=20.0):
    """The reference's CPU fallback (hy_nomas/ops.py:172-176: dequantize the g128 int8 weight to bf16, then
    F.linear) on a row sample of the four GEMMs; rows are scaled so the timed work is ~target_s.  Beside it,
    the single W8A8 linear of the CPU workload (1024 x 3072 -> 3072) through the same fallback and through
    the oracle's W8A8 restatement, and torch's elementwise forms."""
    import oracle

    host = cpu_host()
    threads = max(1, min(host["affinity_cpus"], CPU_SHARE))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    layers = []
    for name, k, n in STACK:
        w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        sw = torch.rand(n, k // 128, generator=g) * 4e-3 + 1e-3
        bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
        layers.append((k, n, w, sw, bias))

    def run(rows):
        t0 = time.perf_counter()
        for k, n, w, sw, bias in layers:
            x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
            oracle.dequant_linear(x, w, sw, bias)
        return time.perf_counter() - t0

    run(64)                          # thread pool and allocator warm-up
    probe = 512
    dt = run(probe)                  # sizes the sample: three passes of about target_s / 3 each
    rows = int(max(64, min(M, probe * target_s / 3 / max(dt, 1e-3))))
    reps = 3
    times = [run(rows) for _ in range(reps)]
    dt = sorted(times)[len(times) // 2]
    ops = sum(2 * rows * n * k for _, k, n in STACK)
    return {"value": round(ops / dt / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{rows} token rows of each of the 4 GEMMs (M=32768 full), median of {reps}, "
                      f"{dt:.2f} s per pass; dequantize_g128 + bf16 F.linear (the reference's CPU fallback), "
                      f"{threads} threads (this job's CPU share) on {host['cpu_model']}",
            "host": host, "config0": cpu_config0(), "also": cpu_restatements(threads)}


def cpu_config0():
    """The single W8A8 linear of the CPU workload (x bf16 [1024, 3072] with 1 % outlier channels x20, int8
    weights [3072, 3072] with per-channel scales, bias; seed 0), median of 10 after 3 warm-ups: the
    reference's fallback (dequantize + bf16 F.linear; it does not quantize activations) and the oracle's W8A8
    restatement (per-token half-even quantization, exact integer products, dequantization + bias)."""
    import oracle

    m, k, n = 1024, HIDDEN, HIDDEN
    g = torch.Generator().manual_seed(0)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[: k // 100]] *= 20
    x = x.to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    sw = (torch.rand(n, 1, generator=g) * 4e-3 + 1e-3).float()
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    wn, swn, bn = w.numpy(), sw.numpy(), oracle.to_f32(bias)

    def w8a8():
        qa, sa = oracle.quantize(x, k, "int8", rounding="half_even")
        return oracle.block_gemm(qa, sa, wn, swn, bn)

    out = {}
    ops = 2 * m * n * k
    for name, fn in (("reference_fallback", lambda: oracle.dequant_linear(x, w, sw, bias)), ("w8a8_oracle", w8a8)):
        for _ in range(3):
            fn()
        ts = []
        for _ in range(10):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        t = sorted(ts)[len(ts) // 2]
        out[name] = {"ms": round(t * 1e3, 3), "TOPS": round(ops / t / 1e12, 4)}
    return out


def cpu_restatements(threads):
    """The arithmetic of the path restated on the CPU, timed beside the fallback: the oracle's g128
    activation quantizer and the torch forms of adaLN and the gated residual at [1, 32768, 3072] (median of 3
    each, one for the quantizer)."""
    import oracle

    g = torch.Generator().manual_seed(1)

    def med(fn, reps=3):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[reps // 2]

    big = torch.randn(1, M, HIDDEN, generator=g).to(torch.bfloat16)
    y = torch.randn(1, M, HIDDEN, generator=g).to(torch.bfloat16)
    shift = (torch.randn(1, HIDDEN, generator=g) * 0.1).to(torch.bfloat16)
    scale = (torch.randn(1, HIDDEN, generator=g) * 0.1).to(torch.bfloat16)
    gate = (torch.randn(1, HIDDEN, generator=g) * 0.1).to(torch.bfloat16)
    t_quant = med(lambda: oracle.quantize(big.view(M, HIDDEN)), 1)
    t_adaln = med(lambda: (torch.nn.functional.layer_norm(big.float(), (HIDDEN,), eps=1e-6)
                           * (1 + scale.float()).to(torch.bfloat16).float()[:, None] + shift.float()[:, None])
                  .to(torch.bfloat16))
    t_gr = med(lambda: big + y * gate[:, None])
    n_el = M * HIDDEN
    return {"threads": threads,
            "quantize_g128_oracle_GBps": round(n_el * (3 + 4 / 128) / t_quant / 1e9, 2),
            "adaln_torch_GBps": round(n_el * 4 / t_adaln / 1e9, 2),
            "gated_residual_torch_GBps": round(n_el * 6 / t_gr / 1e9, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--block-only", action="store_true", help="only the DiT block forward (both layouts)")
    ap.add_argument("--only", choices=["fp8", "g128", "elementwise", "peaks", "refshapes", "config0", "attention"],
                    help="only one of the extra measurements (for per-kernel profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of 512 MiB five times (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the quantized linear path is single-GPU here (token-parallel "
              "sharding needs no exchange between GPUs). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    if args.calibrate_copy:
        src = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel(), "copy_bytes_written": dst.numel(), "launches": 5}))
        return

    if args.only == "fp8":
        ms_f, per_f, ops = gemm_stack(dev, gen, args.steps, args.warmup, kind="fp8")
        print(json.dumps({"fp8_block_gemm_stack_ms": round(ms_f, 4), "per_gemm_ms": [round(t, 4) for t in per_f],
                          "TFLOPS": round(ops / (ms_f * 1e-3) / 1e12, 1)}))
        print(json.dumps({"decoder_mlp_fp8": decoder_mlp(dev, gen, args.steps, args.warmup)}))
        return
    if args.only == "g128":
        ms_g, per_g, ops = gemm_stack(dev, gen, args.steps, args.warmup, group_mode="g128")
        print(json.dumps({"int8_g128_stack_ms": round(ms_g, 4), "per_gemm_ms": [round(t, 4) for t in per_g],
                          "TOPS": round(ops / (ms_g * 1e-3) / 1e12, 1)}))
        return
    if args.only == "peaks":
        print(json.dumps({"peaks": peaks(dev, gen)}))
        return
    if args.only == "refshapes":
        print(json.dumps({"reference_shapes": reference_shapes(dev, gen, max(5, args.steps // 2), 2)}))
        return
    if args.only == "config0":
        print(json.dumps({"config0_gpu": config0_gpu(dev, args.steps, args.warmup)}))
        return
    if args.only == "attention":
        print(json.dumps({"attention": attention_only(dev, gen, max(3, args.steps // 4), 1)}))
        return
    if args.only == "elementwise":
        print(json.dumps(elementwise(dev, gen, max(10, args.steps), 3)))
        print(json.dumps(kv_history(dev, gen, max(10, args.steps), 3)))
        print(json.dumps({"modulation_linear": modulation_linear(dev, gen, max(10, args.steps), 3)}))
        return
    if args.block_only:
        with torch.no_grad():
            print(json.dumps({("per_token" if pt else "g128"): dit_block(dev, gen, 3, 1, pt) for pt in (True, False)}))
        return

    log("bench: int8 per-token x per-channel stack")
    ms, per, ops = gemm_stack(dev, gen, args.steps, args.warmup)
    value = ops / (ms * 1e-3) / 1e12
    kernel_ms = sum(per)
    achieved = ops / (kernel_ms * 1e-3) / 1e12
    per_gemm = {name: {"ms": round(t, 4), "TOPS": round(2 * M * n * k / (t * 1e-3) / 1e12, 1)}
                for (name, k, n), t in zip(STACK, per)}
    result = {
        "metric": "W8A8 GEMM TOPS & % int8 MFMA peak; DiT-block linear-stack ms at M=32768",
        "value": round(value, 1),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "DiT-block W8A8 linear stack, M=32768 tokens, hidden 3072: QKV 3072->9216, "
                               "attn-out 3072->3072, FFN-up 3072->12288, FFN-down 12288->3072; per-token int8 "
                               "activations x per-channel int8 weights, bf16 bias, bf16 out",
                   "M": M, "hidden": HIDDEN, "ops_per_step": ops, "frac_int8_peak": round(value / PEAK_INT8_TOPS, 3)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": round(achieved / PEAK_INT8_TOPS, 3), "traffic": TRAFFIC_BYTES_PER_STEP / len(STACK),
                     "traffic_unit": "bytes per launch, the average of the four GEMMs of a step (rocprofv3 "
                                     "FETCH_SIZE x2.0 + WRITE_SIZE x1.0 per launch; FETCH_SIZE includes "
                                     "Infinity Cache hits)",
                     "kernel": "block_gemm_kernel (int8, per-token)", "per_gemm": per_gemm},
    }
    if not args.no_extra:
        extra = {}
        log("bench: stack with activation quantization")
        ms_q = linear_stack_with_quant(dev, gen, max(5, args.steps // 2), 2)
        extra["linear_stack_with_act_quant"] = {"ms": round(ms_q, 4), "TOPS": round(ops / (ms_q * 1e-3) / 1e12, 1)}
        log("bench: int8 g128 stack")
        ms_g, per_g, _ = gemm_stack(dev, gen, max(5, args.steps // 2), 2, group_mode="g128")
        extra["int8_g128_stack"] = {"ms": round(ms_g, 4), "TOPS": round(ops / (ms_g * 1e-3) / 1e12, 1),
                                    "frac_int8_peak": round(ops / (ms_g * 1e-3) / 1e12 / PEAK_INT8_TOPS, 3),
                                    "per_gemm_ms": [round(t, 4) for t in per_g]}
        log("bench: fp8 block-scaled stack")
        ms_f, per_f, _ = gemm_stack(dev, gen, max(5, args.steps // 2), 2, kind="fp8")
        fp8 = {}
        for (name, k, n), t in zip(STACK, per_f):
            fp8[name] = {"ms": round(t, 4), "TFLOPS": round(2 * M * n * k / (t * 1e-3) / 1e12, 1)}
        extra["fp8_block_gemm"] = {"per_gemm": fp8, "stack_ms": round(ms_f, 4),
                                   "frac_fp8_peak": round(ops / (ms_f * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 3)}
        log("bench: fp8 stack, block scales expanded per channel (the reference's layout)")
        ms_e, per_e, _ = gemm_stack(dev, gen, max(5, args.steps // 2), 2, kind="fp8", expand=True)
        extra["fp8_expanded_scales"] = {"stack_ms": round(ms_e, 4), "TFLOPS": round(ops / (ms_e * 1e-3) / 1e12, 1),
                                        "per_gemm_ms": [round(t, 4) for t in per_e]}
        log("bench: decoder MLP (fp8, fused SwiGLU)")
        extra["decoder_mlp_fp8"] = decoder_mlp(dev, gen, max(5, args.steps // 2), 2)
        log("bench: elementwise")
        extra["elementwise"] = elementwise(dev, gen, max(10, args.steps), 3)
        log("bench: kv history")
        extra["kv_history"] = kv_history(dev, gen, max(10, args.steps), 3)
        log("bench: modulation linear (M = batch)")
        extra["modulation_linear"] = modulation_linear(dev, gen, max(10, args.steps), 3)
        for pt in (True, False):
            name = "dit_block_M57344_" + ("per_token" if pt else "g128")
            log("bench: " + name)
            try:
                extra[name] = dit_block(dev, gen, 3, 1, pt)
            except RuntimeError as e:  # e.g. no flash / memory-efficient SDPA kernel for this device
                extra[name] = {"error": str(e)[:200]}
        log("bench: the reference benchmark's shapes (g128 int8, fp8 blocks, bf16)")
        extra["reference_shapes"] = reference_shapes(dev, gen, max(5, args.steps // 2), 2)
        log("bench: peak probes")
        extra["peaks"] = peaks(dev, gen)
        result["roofline"]["measured_ceiling"] = {
            "int8_mfma_TOPS": extra["peaks"]["int8_mfma"]["TOPS"],
            "frac_of_measured": round(achieved / extra["peaks"]["int8_mfma"]["TOPS"], 3),
            "note": "MFMA loop on real operand data at the power-limited clock (extra.peaks); frac stays "
                    "against the published peak"}
        result["extra"] = extra
    if not args.no_cpu:
        log("bench: config 0 on the GPU")
        gpu0 = config0_gpu(dev, args.steps, args.warmup)
        log("bench: cpu baseline")
        result["cpu_baseline"] = cpu_baseline()
        result["cpu_baseline"]["config0"]["gpu"] = gpu0
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
