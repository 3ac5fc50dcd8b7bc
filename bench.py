#!/usr/bin/env python3
"""Benchmark of the fused attention operator on one MI355X.

A step is one simulated DiT denoising step of the batch-64 throughput sweep: 14 blocks x
(self-attention 64 x 9 heads x 256 x 64, then cross-attention with per-sequence key lengths
~ U{1..128}), each block with its own device-resident inputs. `value` is the whole sweep's
sustained fp32 TFLOP/s (FLOPs = 4*D per attended query/key pair, app/gpu/ops.js:116).

The same JSON line carries:
  headline     DiT self-attention batch 2 x 9 x 256 x 64: us/call, TFLOP/s, fraction of peak
  per_config   us/call and TFLOP/s of the four single-call configs (DiT self and cross at batch 2, T5,
               VAE), each with the PyTorch fp32 CPU time of the same call on all host threads, the
               speed-up, and the GPU output's rel-L2 / normwise max relative error against it
  roofline     the dominant kernel (sweep self-attention), timed per launch with HIP events
  cpu_baseline the PyTorch fp32 CPU formulation of tools/reference.py:72-79 on a bounded sample
  callsite / linear / vae_block / weights  the callers and data either side of the operator: batched
               DiT call sites, the DiT linears, the VAE mid-block in one call, the safetensors loader

    python bench.py [--steps 50] [--warmup 20] [--cpu-seconds 12] [--no-cpu]

`--profile WORKLOAD` instead launches one workload (sweep_self, sweep_cross or a single-call
config) `--launches` times, then copies a 256 MiB device buffer 4 times with the runtime's copy
kernel: a short program for rocprofv3 counter passes, whose per-dispatch FETCH_SIZE/WRITE_SIZE of
the copy (known bytes) calibrate the attention kernel's HBM traffic.

`--summarize RUN_DIR --workloads a,b --out profiles/X.md --title T --trace-cmd C --pmc-cmd C`
turns such passes into a profile summary (no GPU needed): RUN_DIR/trace holds the
`rocprofv3 --kernel-trace --stats -o bench` CSVs of a benchmark run, RUN_DIR/pmc_<workload>_<first
counter>/run_counter_collection.csv the counter passes of `--profile <workload>` (FETCH_SIZE,
WRITE_SIZE, and SQ_VALU_MFMA_BUSY_CYCLES with the other SQ/GRBM counters of the table). The HBM
bytes per launch of every workload go to profiles/hbm_traffic.json, stamped with the digest of the
kernel sources, which `roofline.traffic` reads back.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "supra2-img-web_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fused-attn µs/call + TFLOP/s (DiT 2×9×256×64 fp32), % of fp32 MFMA peak"
PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    sys.stderr.write(f"[bench {time.strftime('%H:%M:%S')}] {msg}\n")
    sys.stderr.flush()


MIN_WARMUP_S = 0.05  # the GPU clocks take about 25 ms of load to settle; every timing warms up at least this long


def warm(dev, launch, calls: int, seconds: float = MIN_WARMUP_S) -> None:
    """At least `calls` calls and at least `seconds` of device time of back-to-back calls."""
    for _ in range(calls):
        launch()
    dev.sync()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            launch()
        dev.sync()


def time_calls(dev, launch, n: int, warmup: int) -> float:
    """Average ms per call of `launch` over n back-to-back calls on the device stream, after a
    warm-up of `warmup` calls and at least MIN_WARMUP_S of calls."""
    from supra_attn.device import Event

    warm(dev, launch, warmup)
    e0, e1 = Event(), Event()
    e0.record(dev.stream)
    for _ in range(n):
        launch()
    e1.record(dev.stream)
    dev.sync()
    return e0.elapsed_ms(e1) / n


def kernel_sources_digest() -> str:
    """sha256 of every kernel and C ABI source (csrc/*.hip, csrc/*.h, include/*.h), in name order:
    the counter figures in profiles/hbm_traffic.json hold only for the sources they were measured on."""
    import hashlib

    h = hashlib.sha256()
    csrc = os.path.join(PKG, "csrc")
    inc = os.path.join(ROOT, "include")
    files = sorted(os.path.join(csrc, f) for f in os.listdir(csrc) if f.endswith((".hip", ".h")))
    files += sorted(os.path.join(inc, f) for f in os.listdir(inc) if f.endswith(".h"))
    for path in files:
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def traffic_from_profiles(workload: str):
    """HBM bytes per launch of `workload`'s kernel from the committed rocprofv3 counter summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a 256 MiB copy), or None when there is none for the
    current kernel sources (the summary's source digest differs: the kernels changed since)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    if data.get("sources_sha256") != kernel_sources_digest():
        log("profiles/hbm_traffic.json was measured on other kernel sources: traffic reported as null")
        return None
    return data.get(workload, {}).get("bytes_per_launch")


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(data, seconds: float) -> dict:
    """PyTorch fp32 CPU on whole sweep steps (28 calls each), the tools/reference.py formulation,
    inputs already in host memory, repeated until `seconds` of CPU work have been timed."""
    import torch

    from oracle import attention as orc

    threads = torch.get_num_threads()
    blocks = [data.block(i) for i in range(data.blocks)]
    flops = sum(s.flops() + c.flops() for s, c in blocks)
    # warm-up call
    orc.cpu_dit_self(blocks[0][0])
    t0 = time.perf_counter()
    steps, last = 0, t0
    while True:
        for s, c in blocks:
            orc.cpu_dit_self(s)
            orc.cpu_dit_cross(c)
        steps += 1
        now = time.perf_counter()
        if now - t0 >= seconds:
            break
        if now - last >= 5.0:
            log(f"cpu baseline: {steps} steps in {now - t0:.1f} s")
            last = now
    dt = time.perf_counter() - t0
    return {
        "value": flops * steps / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{steps} of the sweep's denoising steps ({28 * steps} calls: 14 blocks x self+cross, batch 64) "
                  f"with torch {torch.__version__} F.scaled_dot_product_attention on the CPU "
                  f"({os.cpu_count()} logical CPUs visible, {threads} threads, {cpu_model()}); "
                  f"{dt:.2f} s, {dt / steps * 1e3:.1f} ms/step",
        "ms_per_step": dt / steps * 1e3,
    }


def config_cpu_leg(name: str, call, gpu_out, min_reps: int = 5, min_seconds: float = 0.5) -> dict:
    """One single-call config on the CPU, as the reference's oracle runs it: PyTorch fp32 on all host
    threads, inputs already in host memory, the tools/reference.py:72-79 formulation on the DiT
    callers' packed layouts (cpu_dit_self / cpu_dit_cross) and the PyTorch fp32 path on the gathered
    heads for T5 (HF T5 eager: bias + additive key mask) and the VAE call (SDPA). Warm-up call, then
    the median of at least `min_reps` calls and `min_seconds`. Also the GPU output's rel-L2 and
    normwise max relative error against that CPU output (tools/check.js:31-44)."""
    import torch

    from oracle import attention as orc

    B, H, D, Lq = call.B, call.H, call.D, call.Lq
    if name.startswith("dit_self"):
        fn = lambda: orc.cpu_dit_self(call).numpy().reshape(B, Lq, H, D)  # noqa: E731
    elif name.startswith("dit_cross"):
        fn = lambda: orc.cpu_dit_cross(call).numpy().reshape(B, Lq, H, D)  # noqa: E731
    else:
        Q, K, V, bias, valid = orc.gather_call(call)
        fn = lambda: orc.attention_torch_fp32(Q, K, V, scale=call.scale, bias=bias, valid=valid)  # noqa: E731
    ref = fn()
    ts = []
    t_end = time.perf_counter() + min_seconds
    while len(ts) < min_reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        ref = fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    dt = ts[len(ts) // 2]
    e = orc.errors(orc.output_view(gpu_out, call), ref)
    return {"cpu_us_per_call": dt * 1e6, "cpu_tflops": call.flops() / dt / 1e12, "cpu_reps": len(ts),
            "cpu_threads": torch.get_num_threads(), "rel_l2_vs_cpu": e["rel_l2"], "max_rel_vs_cpu": e["max_rel"]}


def callsite_block(dev, s_st, c_st, reps: int = 20) -> dict:
    """One DiT block's attention at batch B issued as app/models/dit.js:169-185 issues it (one launch
    per sample: B self-attention calls on the packed qkv, then B cross-attention calls at each
    sample's true key length) against the two batched launches, on the same device-resident inputs."""
    import ctypes

    from supra_attn import _lib
    from supra_attn.device import Event

    sa, ca = s_st.args, c_st.args
    B = sa.B
    key_len = c_st.call.key_len
    per = []
    for a, lens in ((sa, None), (ca, key_len)):
        for b in range(B):
            per.append(_lib.AttnArgs(
                B=1, H=a.H, D=a.D, Lq=a.Lq, Lk=a.Lk if lens is None else int(lens[b]), q=a.q, k=a.k, v=a.v, o=a.o,
                q_off=a.q_off + b * a.sq, k_off=a.k_off + b * a.sk, v_off=a.v_off + b * a.sv, o_off=a.o_off + b * a.so,
                ldq=a.ldq, ldk=a.ldk, ldv=a.ldv, ldo=a.ldo, scale=a.scale))
    lib = _lib.load()
    stream = ctypes.c_void_p(dev.stream)
    refs = [ctypes.byref(a) for a in per]

    def loop():
        for r in refs:
            rc = lib.sa_attention_f32(r, stream)
            if rc:
                _lib.check(rc)

    def batched():
        s_st.launch()
        c_st.launch()

    out = {"workload": f"one DiT block's attention at batch {B}: self + cross (sweep block 0)"}
    for name, fn, n in (("per_sample", loop, len(per)), ("batched", batched, 2)):
        ms = time_calls(dev, fn, reps, warmup=3)
        out[f"{name}_us"] = round(ms * 1e3, 2)
        out[f"{name}_launches"] = n
    out["speedup"] = round(out["per_sample_us"] / out["batched_us"], 2)
    return out


def linear_block(dev, B: int = 64, reps: int = 20, cpu: bool = True) -> dict:
    """The six linears of one DiT block at batch B (app/models/dit.js:167-193: qkv, proj, q, cproj,
    fc1, fc2 at B*256 rows) through sa_linear_f32: per-layer us, TFLOP/s and kernel, and the block
    total; with cpu, the PyTorch fp32 CPU time of the same block (torch.mm + epilogue)."""
    from supra_attn.linear_workloads import dit_block_linears
    from supra_attn.runner import StagedLinear

    calls = dit_block_linears(B=B)
    staged = [StagedLinear(dev, c) for c in calls]
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.1:  # clocks settle
        for st in staged:
            st.launch()
        dev.sync()
    layers = {}
    total_us = 0.0
    for st in staged:
        ms = time_calls(dev, st.launch, reps, warmup=2)
        tf = st.call.flops() / (ms * 1e-3) / 1e12
        total_us += ms * 1e3
        layers[st.call.name] = {"shape": [st.call.M, st.call.N, st.call.K], "kernel": st.kernel,
                                "us": round(ms * 1e3, 2), "tflops": round(tf, 2), "frac_peak": round(tf / PEAK_TFLOPS, 4)}
    for st in staged:
        st.release()
    flops = sum(c.flops() for c in calls)
    out = {"workload": f"one DiT block's linears at batch {B} ({B * 256} rows): qkv, proj (gated residual), q, "
                       "cproj (residual), fc1 (GELU tanh), fc2 (gated residual)",
           "layers": layers, "block_us": round(total_us, 2),
           "block_tflops": round(flops / (total_us * 1e-6) / 1e12, 2),
           "block_frac_peak": round(flops / (total_us * 1e-6) / 1e12 / PEAK_TFLOPS, 4)}
    if cpu:
        import torch

        from oracle import linear as ol

        t0 = time.perf_counter()
        for c in calls:
            ol.linear_torch_fp32(c.x, c.w, c.y0, **c.oracle_kwargs())
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"ms_per_block": round(dt * 1e3, 1), "tflops": round(flops / dt / 1e12, 4),
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "one block (6 layers) through oracle.linear.linear_torch_fp32 (torch.mm)"}
    return out


def vae_block_timing(dev, calls: int = 200) -> dict:
    """The SD-VAE mid-block attention as one call (app/models/vae.js:77-94) at a 32x32 latent."""
    from supra_attn.linear_workloads import vae_block
    from supra_attn.runner import StagedVae

    call = vae_block()
    st = StagedVae(dev, call, in_place=False)
    ms = time_calls(dev, st.launch, calls, warmup=10)
    st.release()
    tf = call.flops() / (ms * 1e-3) / 1e12
    return {"workload": f"VAE mid-block attention, {call.HW} pixels x {call.C} channels: GroupNorm, q|k|v, "
                        "attention, output projection + residual in one call",
            "us_per_call": round(ms * 1e3, 2), "tflops": round(tf, 2), "frac_peak": round(tf / PEAK_TFLOPS, 4),
            "flops_per_call": call.flops()}


def dit_checkpoint() -> dict:
    """The DiT weight file's float32 tensors (app/models/dit.js:67-104, names as
    tools/build_models.py writes them), seeded N(0, 1/K): 14 blocks of adaLN + seven linears, plus
    the embeddings and the final layer."""
    import numpy as np

    D, F, depth = 576, 2304, 14
    rng = np.random.default_rng(50)
    pool = rng.standard_normal(1 << 22, dtype=np.float32)  # windows of one seeded pool (fast to build)
    t = {}

    def draw(shape, scale):
        n = int(np.prod(shape))  # every tensor here is smaller than the pool
        start = int(rng.integers(0, pool.size - n + 1))
        return (pool[start:start + n] * np.float32(scale)).reshape(shape)

    def lin(name, n, k):
        t[name + "weight"] = draw((n, k), 1 / np.sqrt(k))
        t[name + "bias"] = draw((n,), 0.1)

    lin("x_embed.", D, 16)
    lin("t_embed.mlp.0.", D, 256)
    lin("t_embed.mlp.2.", D, D)
    lin("ctx_proj.", D, 768)
    t["pos_embed"] = draw((1, 256, D), 1.0)
    for i in range(depth):
        p = f"blocks.{i}."
        for name, n, k in (("adaln.1.", 6 * D, D), ("self_attn.qkv.", 3 * D, D), ("self_attn.proj.", D, D),
                           ("cross_attn.q.", D, D), ("cross_attn.kv.", 2 * D, D), ("cross_attn.proj.", D, D),
                           ("mlp.0.", F, D), ("mlp.2.", D, F)):
            lin(p + name, n, k)
    lin("final.adaln.1.", 2 * D, D)
    lin("final.linear.", 16, D)
    return t


def weights_load(dev, reps: int = 10, cpu: bool = True) -> dict:
    """The safetensors loader (app/weights.js) on a DiT-shaped checkpoint: bulk upload of the data
    section (PCIe-inclusive), the device decode kernels against the HBM roofline, and a whole load
    (open, upload, every tensor decoded into its own buffer) as the model loader issues it."""
    import shutil
    import tempfile

    import numpy as np
    import torch
    from safetensors.numpy import save_file

    from supra_attn import _lib
    from supra_attn.weights import PinnedBuffer, SafeTensors

    lib = _lib.load()
    tensors = dit_checkpoint()
    # the same checkpoint in bfloat16 (round to nearest even through torch), for the decode kernel
    bf16 = {k: torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16) for k, v in tensors.items()}
    tmp = tempfile.mkdtemp(prefix="sa_weights_")
    try:
        f32_path, bf_path = os.path.join(tmp, "dit_f32.safetensors"), os.path.join(tmp, "dit_bf16.safetensors")
        save_file(tensors, f32_path, metadata={"format": "pt"})
        # a BF16 file with the same header layout: written by hand (NumPy has no bfloat16)
        header, off, blobs = {}, 0, []
        for k, v in bf16.items():
            header[k] = {"dtype": "BF16", "shape": list(v.shape), "data_offsets": [off, off + v.nbytes]}
            off += v.nbytes
            blobs.append(v.tobytes())
        hj = json.dumps(header).encode()
        hj += b" " * (-len(hj) % 8)
        with open(bf_path, "wb") as f:
            f.write(len(hj).to_bytes(8, "little") + hj)
            for b in blobs:
                f.write(b)
        n_tensors = len(tensors)
        numel = sum(v.size for v in tensors.values())
        log(f"weights: DiT checkpoint {n_tensors} tensors, {numel} parameters")

        out = {"workload": f"DiT checkpoint ({n_tensors} tensors, {numel} float32 parameters, "
                           f"{4 * numel / 1e6:.1f} MB; the reference ships float32)"}
        st = SafeTensors.open(f32_path)
        nbytes = st.data_bytes
        dst = dev.empty([nbytes], np.uint8)
        pinned = PinnedBuffer(64 << 20)
        for mode in ("staged", "pageable"):
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                _lib.check(lib.sa_st_upload(st._h, 0, nbytes, dst.ptr, pinned.ptr if mode == "staged" else None,
                                            pinned.nbytes if mode == "staged" else 0, dev.stream))
                ts.append(time.perf_counter() - t0)
            out[f"upload_{mode}_gbs"] = round(nbytes / min(ts) / 1e9, 2)
        pinned.release()
        dst.release()
        st.close()

        # decode kernels: the whole data section as one array (BF16 -> f32, F32 -> f32) and the
        # per-tensor launches a model load issues
        with SafeTensors.open(bf_path) as sb:
            res = sb.resident(dev)
            n = sb.data_bytes // 2
            outbuf = dev.empty([n], np.float32)
            launch = lambda: _lib.check(lib.sa_to_f32(res.ptr, _lib.SA_DT["BF16"], n, outbuf.ptr, dev.stream))
            ms = time_calls(dev, launch, reps, warmup=3)
            moved = n * 2 + n * 4
            out["decode_bf16"] = {"elements": n, "us_per_launch": round(ms * 1e3, 2),
                                  "gbs": round(moved / (ms * 1e-3) / 1e9, 1),
                                  "frac_hbm": round(moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                  "bytes_per_launch": moved}
            outbuf2 = dev.empty([n], np.float32)
            launch32 = lambda: _lib.check(lib.sa_to_f32(outbuf.ptr, _lib.SA_DT["F32"], n, outbuf2.ptr, dev.stream))
            ms32 = time_calls(dev, launch32, reps, warmup=3)
            out["decode_f32"] = {"elements": n, "us_per_launch": round(ms32 * 1e3, 2),
                                 "gbs": round(8 * n / (ms32 * 1e-3) / 1e9, 1),
                                 "frac_hbm": round(8 * n / (ms32 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
            outbuf2.release()
            names = sb.names()
            infos = [sb.raw_info(k) for k in names]
            offs = np.cumsum([0] + [int(t.numel) for t in infos])

            def per_tensor():
                for t, o in zip(infos, offs):
                    _lib.check(lib.sa_to_f32(res.ptr + int(t.begin), t.dtype, t.numel, outbuf.ptr + 4 * int(o),
                                             dev.stream))

            ms_pt = time_calls(dev, per_tensor, reps, warmup=2)
            out["decode_bf16_per_tensor"] = {"launches": len(infos), "us_total": round(ms_pt * 1e3, 1),
                                             "gbs": round(moved / (ms_pt * 1e-3) / 1e9, 1)}
            outbuf.release()

        # a whole load as app/models/dit.js issues it: open, bulk upload, one decode per tensor
        # into its own buffer (uploadLinear / uploadVector), synchronized
        dev.sync()
        t0 = time.perf_counter()
        with SafeTensors.open(f32_path) as s2:
            bufs = [s2.f32(dev, k) for k in s2.names()]
            dev.sync()
            load_s = time.perf_counter() - t0
        for b in bufs:
            b.release()
        out["load_ms"] = round(load_s * 1e3, 1)
        out["load_gbs"] = round(4 * numel / load_s / 1e9, 2)
        if cpu:
            # the reference decodes on the CPU (toF32); the oracle's NumPy restatement over the
            # BF16 checkpoint's tensors, all of them (about 0.2 GB of input)
            from oracle import weights as ow

            raw = [v.tobytes() for v in bf16.values()]
            t0 = time.perf_counter()
            for r in raw:
                ow.to_f32(r, "BF16")
            dt = time.perf_counter() - t0
            out["cpu_baseline"] = {"decode_bf16_ms": round(dt * 1e3, 1),
                                   "gbs": round(6 * numel / dt / 1e9, 2), "cores": 1, "kind": "port",
                                   "sample": "every tensor of the BF16 checkpoint through oracle.weights.to_f32"}
        return out
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


COPY_BYTES = 256 << 20


def profile_decode(dev, launches: int) -> int:
    """`launches` BF16 -> float32 decodes of the DiT checkpoint's size (102.5 M elements), then the
    calibration copies."""
    import ctypes

    import numpy as np

    from supra_attn import _lib

    n = sum(v.size for v in dit_checkpoint().values())
    src, dst = dev.empty([n], np.uint16), dev.empty([n], np.float32)
    src.fill_bytes(0x3F)
    log(f"profile weights_bf16: {launches} decodes of {n} elements, {6 * n} algorithmic bytes per launch")
    for _ in range(launches):
        _lib.check(_lib.load().sa_to_f32(src.ptr, _lib.SA_DT["BF16"], n, dst.ptr, dev.stream))
    dev.sync()
    a, b = dev.empty((COPY_BYTES // 4,)), dev.empty((COPY_BYTES // 4,))
    a.fill_bytes(0)
    for _ in range(4):
        _lib.check(_lib.load().sa_memcpy_d2d(b.ptr, a.ptr, COPY_BYTES, ctypes.c_void_p(dev.stream)))
    dev.sync()
    log(f"profile weights_bf16: done ({COPY_BYTES} bytes per calibration copy)")
    return 0


def profile_run(workload: str, launches: int) -> int:
    import ctypes

    from supra_attn import _lib, workloads
    from supra_attn.device import Device
    from supra_attn.runner import Staged

    dev = Device(0)
    if workload == "weights_bf16":
        return profile_decode(dev, launches)
    if workload == "vae_block":
        from supra_attn.linear_workloads import vae_block
        from supra_attn.runner import StagedVae

        call = vae_block()
        st = StagedVae(dev, call)
    elif workload.startswith("linear_"):
        from supra_attn.linear_workloads import dit_block_linears
        from supra_attn.runner import StagedLinear

        call = [c for c in dit_block_linears(B=64) if c.name == workload[len("linear_"):]][0]
        st = StagedLinear(dev, call)
    elif workload in ("sweep_self", "sweep_cross"):
        s, c = workloads.SweepData(blocks=1).block(0)
        call = s if workload == "sweep_self" else c
        st = Staged(dev, call)
    else:
        call = workloads.CONFIGS[workload]()
        st = Staged(dev, call)
    log(f"profile {workload}: {launches} launches of {st.kernel}, "
        f"{call.flops()} flop and {call.algorithmic_bytes()} algorithmic bytes per launch")
    for _ in range(launches):
        st.launch()
    dev.sync()
    src, dst = dev.empty((COPY_BYTES // 4,)), dev.empty((COPY_BYTES // 4,))
    src.fill_bytes(0)
    for _ in range(4):
        _lib.check(_lib.load().sa_memcpy_d2d(dst.ptr, src.ptr, COPY_BYTES, ctypes.c_void_p(dev.stream)))
    dev.sync()
    log(f"profile {workload}: done ({COPY_BYTES} bytes per calibration copy)")
    return 0


def summarize(run: str, workloads: list[str], out_md: str, title: str, trace_cmd: str, pmc_cmd: str,
              trace_filter: str = "") -> int:
    """Profile summary (markdown) of a rocprofv3 run directory, and the HBM bytes per launch of each
    workload into profiles/hbm_traffic.json (see the module docstring for the layout)."""
    import csv
    import glob
    import statistics

    cus, simds, xcds = 256, 1024, 8
    med = statistics.median

    def clean(name: str) -> str:
        return name.replace("(anonymous namespace)::", "").replace("void ", "").replace("sa::", "").split("(")[0]

    lines = [title, "", "Commands (from the repository root on the MI355X box; rocprofv3 run from /tmp with "
             "TMPDIR=/tmp):", "", "```", trace_cmd, pmc_cmd, "```", ""]
    stats_path = os.path.join(run, "trace", "bench_kernel_stats.csv")
    if os.path.exists(stats_path):
        lines += ["## Kernel trace (`--kernel-trace --stats` over the benchmark), average duration per kernel", "",
                  "| kernel | calls | avg us | min us | max us | share |", "|---|---|---|---|---|---|"]
        for r in csv.DictReader(open(stats_path)):
            if trace_filter and trace_filter not in r["Name"]:
                continue
            lines.append(f"| `{clean(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f}% |")
        groups: dict = {}
        for r in csv.DictReader(open(os.path.join(run, "trace", "bench_kernel_trace.csv"))):
            if "sa::" not in r["Kernel_Name"] or (trace_filter and trace_filter not in r["Kernel_Name"]):
                continue
            key = (clean(r["Kernel_Name"]), int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]))
            groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        lines += ["", "### The same trace by launch shape (workgroups per launch)", "",
                  "| kernel | workgroups | calls | avg us | min us | max us |", "|---|---|---|---|---|---|"]
        for (k, wg), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:14]:
            lines.append(f"| `{k}` | {wg} | {len(d)} | {sum(d) / len(d):.1f} | {min(d):.1f} | {max(d):.1f} |")
    pmc: dict = {}
    for f in sorted(glob.glob(os.path.join(run, "pmc_*", "run_counter_collection.csv"))):
        tag = os.path.basename(os.path.dirname(f))[4:]
        wl = next((w for w in workloads if tag.startswith(w + "_")), None)
        if wl is None:
            continue
        for r in csv.DictReader(open(f)):
            name = r["Kernel_Name"]
            if "copyBuffer" in name and int(r["Grid_Size"]) > 100000:
                key = "copy"
            elif "sa::" in name:
                key = clean(name)
            else:
                continue
            d = pmc.setdefault(wl, {}).setdefault(key, {})
            d.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            d.setdefault("dur", []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines += ["", "## Counters per dispatch (median over the launches); HBM bytes calibrated with a 256 MiB copy", "",
              "| workload | kernel | avg us (counter runs) | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM MB (cal.) | "
              "MFMA FLOP (MOPS_F32 x 512) | MFMA busy | LDS bank conflicts / LDS active | mean waves/CU |",
              "|---|---|---|---|---|---|---|---|---|---|"]
    tj = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    traffic = {}
    if os.path.exists(tj):
        with open(tj) as f:
            traffic = json.load(f)
        if traffic.get("sources_sha256") != kernel_sources_digest():
            traffic = {}  # figures of other kernel sources are dropped, not mixed in
    cal = None
    for wl in workloads:
        d = pmc.get(wl)
        if not d or "copy" not in d:
            print(f"no counter passes for {wl} under {run}", file=sys.stderr)
            return 1
        c = d["copy"]
        fcal = COPY_BYTES / 1024 / med(c["FETCH_SIZE"])
        wcal = COPY_BYTES / 1024 / med(c["WRITE_SIZE"])
        cal = cal or (med(c["FETCH_SIZE"]), med(c["WRITE_SIZE"]))
        total = 0.0
        for k, a in d.items():
            if k == "copy":
                continue
            fetch, write = med(a["FETCH_SIZE"]), med(a["WRITE_SIZE"])
            hbm = (fetch * fcal + write * wcal) * 1024
            total += hbm
            if "GRBM_GUI_ACTIVE" in a:
                grbm = med(a["GRBM_GUI_ACTIVE"]) / xcds
                util = f"{100 * med(a['SQ_VALU_MFMA_BUSY_CYCLES']) / simds / grbm:.1f}%"
                mops = f"{med(a['SQ_INSTS_VALU_MFMA_MOPS_F32']) * 512:.4g}"
                lds = f"{med(a['SQ_LDS_BANK_CONFLICT']):.0f} / {med(a['SQ_LDS_IDX_ACTIVE']):.0f}"
                waves = f"{4 * med(a['SQ_WAVE_CYCLES']) / grbm / cus:.1f}"
            else:
                util = mops = lds = waves = "-"
            lines.append(f"| {wl} | `{k}` | {med(a['dur']):.1f} | {fetch:.0f} | {write:.0f} | {hbm / 1e6:.1f} | "
                         f"{mops} | {util} | {lds} | {waves} |")
        traffic[wl] = {"kernels": [k for k in d if k != "copy"], "bytes_per_launch": round(total),
                       "fetch_factor": round(fcal, 4), "write_factor": round(wcal, 4)}
    lines += ["", f"Calibration: the runtime's copy kernel moving {COPY_BYTES} bytes reads FETCH_SIZE = {cal[0]:.1f} KiB "
              f"and WRITE_SIZE = {cal[1]:.1f} KiB per dispatch, so HBM bytes = FETCH_SIZE x 1024 x "
              f"{COPY_BYTES / 1024 / cal[0]:.3f} + WRITE_SIZE x 1024 x {COPY_BYTES / 1024 / cal[1]:.3f}.",
              "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM_GUI_ACTIVE / 8 XCDs); mean waves/CU = "
              "4 x SQ_WAVE_CYCLES / (GRBM_GUI_ACTIVE / 8) / 256.",
              f"Kernel sources: sha256 {kernel_sources_digest()[:16]}... (`bench.py` `kernel_sources_digest`).", ""]
    with open(out_md, "w") as f:
        f.write("\n".join(lines))
    traffic["sources_sha256"] = kernel_sources_digest()
    with open(tj, "w") as f:
        json.dump(traffic, f, indent=1, sort_keys=True)
    print("\n".join(lines))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)  # plus at least MIN_WARMUP_S of steps: the clocks settle after ~25 ms
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calls", type=int, default=200, help="calls per single-config timing")
    ap.add_argument("--profile", default=None, help="launch only this workload (for rocprofv3 counter passes)")
    ap.add_argument("--launches", type=int, default=20)
    ap.add_argument("--summarize", default=None, metavar="RUN_DIR", help="write a profile summary (no GPU)")
    ap.add_argument("--workloads", default="", help="--summarize: comma-separated workloads of the counter passes")
    ap.add_argument("--out", default=None, help="--summarize: the markdown file to write")
    ap.add_argument("--title", default="", help="--summarize: first line of the summary")
    ap.add_argument("--trace-cmd", default="", help="--summarize: the kernel-trace command, quoted in the summary")
    ap.add_argument("--pmc-cmd", default="", help="--summarize: the counter-pass command, quoted in the summary")
    ap.add_argument("--trace-filter", default="", help="--summarize: keep trace rows whose kernel name has this")
    args = ap.parse_args()
    if args.summarize:
        return summarize(args.summarize, [w for w in args.workloads.split(",") if w], args.out, args.title,
                         args.trace_cmd, args.pmc_cmd, args.trace_filter)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this operator's path has no multi-GPU form here (asked for --gpus {args.gpus}); "
              "the per-GPU shard of a sharded run is the same kernel at the shapes measured with --gpus 1.",
              file=sys.stderr)
        return 2
    if args.profile:
        return profile_run(args.profile, args.launches)

    from supra_attn import workloads
    from supra_attn.device import Device, Event
    from supra_attn.runner import Staged

    dev = Device(0)
    log("generating sweep inputs")
    data = workloads.SweepData()
    staged = []
    for i in range(data.blocks):
        s, c = data.block(i)
        staged.append((Staged(dev, s), Staged(dev, c)))
    dev.sync()
    self_kernel = staged[0][0].kernel
    cross_kernel = staged[0][1].kernel
    step_flops = sum(s.call.flops() + c.call.flops() for s, c in staged)
    log(f"sweep staged: {data.blocks} blocks, self={self_kernel}, cross={cross_kernel}, "
        f"{step_flops / 1e9:.2f} GFLOP/step")

    def step():
        for s, c in staged:
            s.launch()
            c.launch()

    warm(dev, step, args.warmup)  # --warmup steps, and at least MIN_WARMUP_S of them
    e0, e1 = Event(), Event()
    e0.record(dev.stream)
    for _ in range(args.steps):
        step()
    e1.record(dev.stream)
    dev.sync()
    total_ms = e0.elapsed_ms(e1)
    ms_per_step = total_ms / args.steps
    value = step_flops * args.steps / (total_ms * 1e-3) / 1e12
    log(f"sweep: {ms_per_step:.3f} ms/step, {value:.2f} TFLOP/s")

    # Per-launch time of each kernel: the sweep's self-attention calls back to back (the 14 input
    # sets in turn, one event pair over steps x 14 calls), then its cross-attention calls likewise.
    # Launch gaps are included; no event sits between launches.
    def b2b(idx: int) -> float:
        for pair in staged:
            pair[idx].launch()
        a, z = Event(), Event()
        a.record(dev.stream)
        for _ in range(args.steps):
            for pair in staged:
                pair[idx].launch()
        z.record(dev.stream)
        dev.sync()
        return a.elapsed_ms(z) / (args.steps * data.blocks)

    self_ms = b2b(0)
    cross_ms = b2b(1)
    # the same with an event pair around every launch inside the sweep's alternation (each pair adds
    # its own record overhead to the launch it brackets)
    pairs_s = [(Event(), Event()) for _ in range(args.steps * data.blocks)]
    pairs_c = [(Event(), Event()) for _ in range(args.steps * data.blocks)]
    n = 0
    for _ in range(args.steps):
        for s, c in staged:
            a, b = pairs_s[n]
            a.record(dev.stream)
            s.launch()
            b.record(dev.stream)
            a, b = pairs_c[n]
            a.record(dev.stream)
            c.launch()
            b.record(dev.stream)
            n += 1
    dev.sync()
    self_ms_ev = sum(a.elapsed_ms(b) for a, b in pairs_s) / len(pairs_s)
    cross_ms_ev = sum(a.elapsed_ms(b) for a, b in pairs_c) / len(pairs_c)
    self_call = staged[0][0].call
    self_flops = self_call.flops()
    achieved = self_flops / (self_ms * 1e-3) / 1e12
    cross_flops = sum(c.call.flops() for _, c in staged) / len(staged)
    log(f"per launch: self {self_ms * 1e3:.1f} us ({achieved:.1f} TFLOP/s), cross {cross_ms * 1e3:.1f} us "
        f"(one event pair per launch: {self_ms_ev * 1e3:.1f} / {cross_ms_ev * 1e3:.1f} us)")

    # caller side: per-sample launches (the reference's loops) against the batched call sites
    callsite = callsite_block(dev, staged[0][0], staged[0][1])
    log(f"call sites, one block: per-sample {callsite['per_sample_us']:.1f} us ({callsite['per_sample_launches']} "
        f"launches) vs batched {callsite['batched_us']:.1f} us (2 launches): {callsite['speedup']:.2f}x")

    # the linears either side of attention in the same DiT block
    linear = linear_block(dev, cpu=not args.no_cpu)
    log(f"linears, one block at batch 64: {linear['block_us']:.1f} us, {linear['block_tflops']:.1f} TFLOP/s "
        + " ".join(f"{k} {v['us']:.0f}us" for k, v in linear["layers"].items()))

    # the weight loader feeding those linears (app/weights.js): upload, device decode, whole load
    weights = weights_load(dev, cpu=not args.no_cpu)
    log(f"weights: upload {weights['upload_staged_gbs']} GB/s staged, {weights['upload_pageable_gbs']} GB/s pageable; "
        f"bf16 decode {weights['decode_bf16']['us_per_launch']} us ({weights['decode_bf16']['gbs']} GB/s); "
        f"whole load {weights['load_ms']} ms")

    # single-call configs
    per_config = {}
    for name, make in workloads.CONFIGS.items():
        call = make()
        st = Staged(dev, call)
        ms = time_calls(dev, st.launch, args.calls, warmup=10)
        tf = call.flops() / (ms * 1e-3) / 1e12
        per_config[name] = {
            "kernel": st.kernel,
            "us_per_call": ms * 1e3,
            "tflops": tf,
            "frac_peak": tf / PEAK_TFLOPS,
            "gbs": call.algorithmic_bytes() / (ms * 1e-3) / 1e9,
            "flops_per_call": call.flops(),
            "bytes_per_call": call.algorithmic_bytes(),
        }
        out = st.run()  # one more call, read back for the parity figures
        st.release()
        log(f"{name}: {ms * 1e3:.2f} us/call, {tf:.2f} TFLOP/s via {per_config[name]['kernel']}")
        if not args.no_cpu:
            leg = config_cpu_leg(name, call, out)
            leg["speedup"] = leg["cpu_us_per_call"] / (ms * 1e3)
            per_config[name].update(leg)
            log(f"{name}: cpu {leg['cpu_us_per_call']:.1f} us/call ({leg['cpu_threads']} threads), "
                f"{leg['speedup']:.1f}x; rel_l2 {leg['rel_l2_vs_cpu']:.2e}, max_rel {leg['max_rel_vs_cpu']:.2e}")
    vae = vae_block_timing(dev)
    log(f"vae_block: {vae['us_per_call']:.2f} us/call, {vae['tflops']:.2f} TFLOP/s")
    for s, c in staged:
        s.release()
        c.release()

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline: whole sweep steps for {args.cpu_seconds:g} s")
        cpu = cpu_baseline(data, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']:.4f} TFLOP/s")

    head = per_config["dit_self_b2"]
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) inputs, 14 distinct device-resident input sets",
        "config": {
            "workload": "dit_sweep_b64: 14 blocks x (self 64x9x256x64 + cross 64x9x256x64, key_len~U{1..128}) per step",
            "global_batch": 64,
            "seq_len": 256,
            "heads": 9,
            "head_dim": 64,
            "cross_key_len_sum": int(data.key_len.sum()),
            "gflop_per_step": round(step_flops / 1e9, 4),
            "frac_peak": round(value / PEAK_TFLOPS, 4),
            "parallelism": "single GPU",
        },
        "headline": {
            "workload": "dit_self_b2 (2x9x256x64)",
            "us_per_call": round(head["us_per_call"], 3),
            "tflops": round(head["tflops"], 3),
            "frac_peak": round(head["frac_peak"], 4),
        },
        "roofline": {
            "kernel": self_kernel,
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS, 4),
            "traffic": traffic_from_profiles("sweep_self"),
            "traffic_sources_sha256": kernel_sources_digest(),
            "algorithmic_flops_per_launch": self_flops,
            "algorithmic_bytes_per_launch": self_call.algorithmic_bytes(),
            "us_per_launch": round(self_ms * 1e3, 3),
            "us_per_launch_timing": "back to back, one event pair over steps x 14 launches",
            "us_per_launch_event_pair_each": round(self_ms_ev * 1e3, 3),
            "cross_us_per_launch": round(cross_ms * 1e3, 3),
            "cross_us_per_launch_event_pair_each": round(cross_ms_ev * 1e3, 3),
            "cross_tflops": round(cross_flops / (cross_ms * 1e-3) / 1e12, 3),
        },
        "per_config": {k: {kk: (float(f"{vv:.4g}") if kk.endswith("_vs_cpu") else round(vv, 4) if isinstance(vv, float)
                            else vv) for kk, vv in v.items()}
                       for k, v in per_config.items()},
        "callsite": callsite,
        "linear": linear,
        "vae_block": vae,
        "weights": weights,
        "cpu_baseline": None if cpu is None else {k: (round(v, 6) if isinstance(v, float) else v) for k, v in cpu.items()},
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
