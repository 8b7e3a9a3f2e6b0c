"""Benchmark of the gfx950 SharedDictionaryAttention forward path.

One step = one ``SharedDictionaryAttention`` forward (dictionary
normalization, Q/K/V projection, fused route, flash attention with the map
mix, output projection) on one synthetic batch already resident in HBM, the
same unit of work as the reference's ``benchmarks/benchmark_attention.py``
forward mode.  The default workload is the north-star configuration: preset
a1, x = [8, 512, 512] bf16.  ``--workload c4`` times the
six-layer tied language model instead: a step is one ``DoubleAttentionLM``
forward over [64, 64] token ids, and the per-kernel lines are one layer's.

Prints ONE JSON line (rank 0).  Besides the module throughput it reports the
per-kernel average durations measured with HIP events on the launch stream,
the roofline of the dominant kernel and the fp32 CPU oracle timed on the
host's cores for a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "double-attention_amd"))
sys.path.insert(0, str(REPO))

METRIC = "routed rows/s + attention tokens/s on 1 MI355X; % MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

WORKLOADS = {
    # name: (preset, batch, length, overrides, description)
    "c1": ("a1", 8, 512, {}, "C1 preset a1 SharedDictionaryAttention forward x=[8,512,512]"),
    "c2": ("qk4-s4", 8, 1024, {}, "C2 preset qk4-s4 SharedDictionaryAttention forward x=[8,1024,512]"),
    "c3": ("a1-r512-d1536", 4, 2048, {}, "C3 preset a1-r512-d1536 SharedDictionaryAttention forward x=[4,2048,512]"),
    "c4": ("qk2-s2", 64, 64, {"untied_dictionary": False},
           "C4 DoubleAttentionLM qk2-s2 tied, 6 layers, vocab 2048, ffn 1536, tokens [64,64]"),
    "c5": ("a1", 1, 8192, {}, "C5 preset a1 long-context SharedDictionaryAttention forward x=[1,8192,512]"),
}


# C4 is the language model: a step is one whole LM forward (token ids to
# logits); the per-kernel lines time one layer's attention launches.
LM_VOCAB, LM_LAYERS, LM_FEEDFORWARD = 2048, 6, 1536


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="c1")
    p.add_argument("--dtype", choices=("bf16", "fp16"), default="bf16")
    p.add_argument("--kernel-reps", type=int, default=200, help="launches per per-kernel timing loop")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument(
        "--backward",
        action="store_true",
        help="time the outer attention's native backward at the workload's attention shape instead "
        "(a separate JSON line; not the headline metric)",
    )
    p.add_argument(
        "--copy-mib",
        type=int,
        default=0,
        help="after the measurement, copy a device buffer of this many MiB three times: a kernel of known "
        "traffic that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters",
    )
    p.add_argument(
        "--kernels-only",
        action="store_true",
        help="run only the per-kernel timing loops (each kernel 5 + --kernel-reps launches, in a fixed order) "
        "and the --copy-mib calibration copies: the child run that --collect-counters profiles; with "
        "--backward, only --steps HIP training steps (module, and for c4 the LM), for a kernel trace",
    )
    p.add_argument(
        "--compare-library",
        action="store_true",
        help="instead of the benchmark: the projection and FFN GEMMs of C1-C5 on the library's MFMA GEMM against "
        "torch (hipBLASLt), both replayed from HIP graphs, and the C1-C5 forwards on backend='hip' against "
        "backend='torch' in bf16 on the same GPU (one JSON line; not the headline metric)",
    )
    p.add_argument(
        "--collect-counters",
        action="store_true",
        help="profile a --kernels-only child run of the workload under rocprofv3 --pmc (MFMA, LDS and HBM "
        "counters, one pass per group) and write profiles/counters_<workload>.json and .md",
    )
    return p.parse_args()


def cpu_info() -> dict:
    """``lscpu``'s model name, physical cores and hardware threads of this host."""

    info = {"model": "unknown", "physical_cores": None, "threads": os.cpu_count()}
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        fields = {k.strip(): v.strip() for k, v in fields.items()}
        info["model"] = fields.get("Model name", "unknown")
        cores = int(fields.get("Core(s) per socket", "0")) * int(fields.get("Socket(s)", "0"))
        info["physical_cores"] = cores or None
        info["threads"] = int(fields.get("CPU(s)", info["threads"] or 0)) or info["threads"]
    except Exception:  # noqa: BLE001 - informational only
        pass
    return info


def kernel_source_hash() -> str:
    """SHA-256 over the kernel library's sources (``csrc``): counter tables
    measured on other sources are stale and are not reported."""

    import hashlib

    h = hashlib.sha256()
    for path in sorted((REPO / "double-attention_amd" / "csrc").iterdir()):
        if path.suffix in (".hip", ".h"):
            h.update(path.name.encode())
            h.update(path.read_bytes())
    return h.hexdigest()[:16]


def measured_counters(workload: str) -> dict | None:
    """Per-kernel rocprofv3 counter summary of ``workload`` written by
    ``--collect-counters`` for the current kernel sources, else None."""

    try:
        table = json.loads((REPO / "profiles" / f"counters_{workload}.json").read_text())
    except (OSError, ValueError):
        return None
    if table.get("source_hash") != kernel_source_hash():
        return None
    return table


# rocprofv3 --pmc passes of --collect-counters: at most 8 SQ, 4 TCC (FETCH_SIZE
# takes 3, WRITE_SIZE 2) and 2 GRBM counters per pass.
COUNTER_PASSES = {
    "mfma": ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
             "SQ_INSTS_VALU_MFMA_MOPS_F16"),
    "lds": ("SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_WAIT_INST_LDS", "SQ_WAVE_CYCLES",
            "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_WAIT_ANY"),
    "fetch": ("FETCH_SIZE",),
    "write": ("WRITE_SIZE",),
}
SIMDS = 1024          # MI355X: 256 CUs x 4 SIMDs
COPY_MIB = 256        # calibration copy of the counter runs


def _kernel_label(name: str) -> str:
    for key, label in (("route_kernel", "route"), ("attention_kernel", "attention"), ("attention_short_kernel", "attention"),
                       ("merge", "attention_merge"),
                       ("dict_normalize", "dict_normalize"), ("gemm_kernel", "gemm"), ("copyBuffer", "copy")):
        if key in name:
            return label
    return name.split("(")[0][-60:]


def collect_counters(args: argparse.Namespace) -> None:
    """Profile a ``--kernels-only`` child run under rocprofv3, one pass per
    counter group, and write ``profiles/counters_<workload>.{json,md}``.

    The child launches dict_normalize, qkv_projection, route, attention and
    output_projection 5 + ``--kernel-reps`` times each, in that order, then
    copies a 256 MiB buffer three times.  GEMM dispatches before the first
    route dispatch are the QKV projection, later ones the output projection.
    Derived figures per dispatch:

    * MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs),
      rocprofv3's MfmaUtil (GRBM_GUI_ACTIVE is read per XCD and summed);
    * MFMA flops executed = (MOPS_BF16 + MOPS_F16) x 512, beside the
      kernel's algorithmic flops;
    * LDS bank conflicts per access = SQ_LDS_BANK_CONFLICT /
      (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT);
    * HBM bytes = FETCH_SIZE / f + WRITE_SIZE / w, where f and w are what the
      counters read per byte of the calibration copy.
    """

    import csv
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    child = [sys.executable, str(REPO / "bench.py"), "--workload", args.workload, "--dtype", args.dtype,
             "--kernels-only", "--kernel-reps", str(min(args.kernel_reps, 20)), "--no-cpu-baseline",
             "--copy-mib", str(COPY_MIB)]
    env = dict(os.environ, TMPDIR="/tmp")
    rows: dict[int, dict] = {}
    commands = []
    for pass_name, counters in COUNTER_PASSES.items():
        out_dir = tempfile.mkdtemp(prefix=f"da_pmc_{pass_name}_", dir="/tmp")
        cmd = ["rocprofv3", "--pmc", *counters, "--kernel-trace", "--output-format", "csv", "-d", out_dir,
               "-o", "run", "--", *child]
        commands.append(" ".join(cmd[:-len(child)] + ["python3", "bench.py", *child[2:]]).replace(out_dir, "<dir>"))
        print(f"[counters] {args.workload} pass {pass_name}: {' '.join(counters)}", file=sys.stderr, flush=True)
        proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                text=True, start_new_session=True)
        try:
            stdout, stderr = proc.communicate(timeout=240)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.communicate()
            raise SystemExit(f"rocprofv3 pass {pass_name} timed out")
        files = glob.glob(f"{out_dir}/**/*counter_collection.csv", recursive=True)
        if not files:
            print(stderr[-3000:], file=sys.stderr)
            raise SystemExit(f"rocprofv3 pass {pass_name} (exit {proc.returncode}) wrote no counter file")
        # A crash after the program's last line with complete results is the
        # profiler's own exit; the counter file is what matters.
        for path in files:
            with open(path, newline="") as f:
                for rec in csv.DictReader(f):
                    d = int(rec["Dispatch_Id"])
                    row = rows.setdefault(d, {"name": rec["Kernel_Name"], "grid": int(rec["Grid_Size"])})
                    row[rec["Counter_Name"]] = row.get(rec["Counter_Name"], 0.0) + float(rec["Counter_Value"])
        shutil.rmtree(out_dir, ignore_errors=True)

    # Label every dispatch; dispatch ids follow launch order within the run.
    first_route = min((d for d, r in rows.items() if _kernel_label(r["name"]) == "route"), default=None)
    groups: dict[str, list[dict]] = {}
    for d, r in sorted(rows.items()):
        label = _kernel_label(r["name"])
        if label == "gemm":
            label = "qkv_projection" if first_route is not None and d < first_route else "output_projection"
        groups.setdefault(label, []).append(r)
    # The calibration copies are the run's last three copies (earlier ones
    # stage the host inputs).
    groups["copy"] = groups.get("copy", [])[-3:]

    def mean(label: str, counter: str) -> float | None:
        vals = [r[counter] for r in groups.get(label, []) if counter in r]
        return sum(vals) / len(vals) if vals else None

    copy_bytes = COPY_MIB << 20
    f_fetch = (mean("copy", "FETCH_SIZE") or 0) * 1024 / copy_bytes
    f_write = (mean("copy", "WRITE_SIZE") or 0) * 1024 / copy_bytes
    xcds = 8
    kernels = {}
    for label, recs in groups.items():
        if label not in ("dict_normalize", "qkv_projection", "route", "attention", "attention_merge",
                         "output_projection"):
            continue
        e = {"dispatches": len(recs), "symbol": recs[0]["name"].split("(")[0][:120]}
        busy, active = mean(label, "SQ_VALU_MFMA_BUSY_CYCLES"), mean(label, "GRBM_GUI_ACTIVE")
        if busy is not None and active:
            e["mfma_busy"] = round(busy / (active / xcds * SIMDS), 4)
        mops = [mean(label, c) for c in ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F16")]
        if all(m is not None for m in mops):
            e["mfma_flops_executed"] = (mops[0] + mops[1]) * 512
        conf, idx = mean(label, "SQ_LDS_BANK_CONFLICT"), mean(label, "SQ_LDS_IDX_ACTIVE")
        if conf is not None and idx and idx > conf:
            e["lds_bank_conflicts_per_access"] = round(conf / (idx - conf), 4)
        wait_lds, wave = mean(label, "SQ_WAIT_INST_LDS"), mean(label, "SQ_WAVE_CYCLES")
        if wait_lds is not None and wave:
            e["lds_issue_wait_frac"] = round(wait_lds / wave, 4)
        wait_any = mean(label, "SQ_WAIT_ANY")
        if wait_any is not None and wave:
            e["wait_any_frac"] = round(wait_any / wave, 4)
        for c in ("SQ_INSTS_LDS", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "FETCH_SIZE", "WRITE_SIZE"):
            v = mean(label, c)
            if v is not None:
                e[c] = round(v, 1)
        fetch, write = mean(label, "FETCH_SIZE"), mean(label, "WRITE_SIZE")
        if fetch is not None and write is not None and f_fetch > 0 and f_write > 0:
            e["hbm_bytes_per_launch"] = round(fetch * 1024 / f_fetch + write * 1024 / f_write)
        kernels[label] = e
    table = {
        "workload": args.workload,
        "dtype": args.dtype,
        "source_hash": kernel_source_hash(),
        "commands": commands,
        "calibration": {"copy_mib": COPY_MIB, "fetch_per_byte": round(f_fetch, 4), "write_per_byte": round(f_write, 4)},
        "kernels": kernels,
    }
    out = REPO / "profiles" / f"counters_{args.workload}.json"
    out.write_text(json.dumps(table, indent=1) + "\n")
    lines = [
        f"# rocprofv3 counters, workload {args.workload} ({WORKLOADS[args.workload][4]}, {args.dtype})",
        "",
        "Written by `python3 bench.py --workload " + args.workload + " --collect-counters` (run from the repository "
        "root; it runs each pass below in /tmp with TMPDIR=/tmp).  Per-dispatch means over every dispatch of each "
        "kernel in a `--kernels-only` child run.  Kernel sources: `" + table["source_hash"] + "` (SHA-256 prefix "
        "of `double-attention_amd/csrc`).",
        "",
        "```",
        *commands,
        "```",
        "",
        f"Calibration: the child copies a {COPY_MIB} MiB buffer three times; per byte moved, FETCH_SIZE reads "
        f"{f_fetch:.3f} and WRITE_SIZE {f_write:.3f} (KiB units), so HBM bytes = FETCH_SIZE*1024/{f_fetch:.3f} + "
        f"WRITE_SIZE*1024/{f_write:.3f}.  MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x "
        f"{SIMDS} SIMDs) (rocprofv3's MfmaUtil); MFMA flops executed = (SQ_INSTS_VALU_MFMA_MOPS_BF16 + _F16) x 512.",
        "",
        "| kernel | dispatches | MFMA busy | MFMA GFLOP executed | LDS conflicts / access | LDS issue wait / wave-cycles "
        "| any wait / wave-cycles | HBM MiB / launch |",
        "|---|---|---|---|---|---|---|---|",
    ]
    for label, e in kernels.items():
        def fmt(key, scale=1.0, digits=3):
            v = e.get(key)
            return "-" if v is None else f"{v * scale:.{digits}f}"
        lines.append(f"| {label} | {e['dispatches']} | {fmt('mfma_busy', 100, 1)}% | {fmt('mfma_flops_executed', 1e-9, 2)} "
                     f"| {fmt('lds_bank_conflicts_per_access')} | {fmt('lds_issue_wait_frac')} | {fmt('wait_any_frac')} "
                     f"| {fmt('hbm_bytes_per_launch', 2 ** -20, 1)} |")
    (REPO / "profiles" / f"counters_{args.workload}.md").write_text("\n".join(lines) + "\n")
    print(json.dumps({"workload": args.workload, "counters": str(out.relative_to(REPO))}), flush=True)


def backward_bench(args: argparse.Namespace) -> None:
    """Outer-attention backward at the workload's attention shape.

    One step = dQ, dK, dV and d(scale) of ``routed_attention_hip`` for one
    output gradient (prep, LSE and key-tile kernels), timed with HIP events
    on the launch stream; beside it the fp32-softmax recompute through torch
    autograd that the backward replaces, and one module training step
    (forward + backward) on the HIP and on the bf16 torch backend.  FLOPs count the five products
    2 T^2 (3R + 2D) per map plus the LSE pass's 2 T^2 R, halved when causal.
    """

    import torch

    import double_attention as da
    from double_attention import hip_ops
    from double_attention.ops import routed_attention_reference

    device = torch.device("cuda:0")
    preset, batch, length, overrides, description = WORKLOADS[args.workload]
    config = da.experiment_config(preset, backend="hip", **overrides)
    H, S, R = config.qk_branches, config.outer_maps, config.routing_dim
    rp = (H // S if H > S else 1) * R
    d = config.model_dim
    g = torch.Generator().manual_seed(3)
    q = torch.nn.functional.normalize(torch.randn(batch, S, length, rp, generator=g), dim=-1).to(device, torch.float16)
    k = torch.nn.functional.normalize(torch.randn(batch, S, length, rp, generator=g), dim=-1).to(device, torch.float16)
    v = torch.randn(batch, length, d, generator=g).to(device, torch.bfloat16)
    scales = torch.full((S,), 8.0, device=device)
    grad = torch.randn(batch, S, length, d, generator=g).to(device, torch.bfloat16)
    causal = config.causal
    out = hip_ops._attention_forward(q, k, v, scales, causal)

    def native():
        # The dispatcher the module backward uses: the dense path for
        # 512-wide scores whose matrices fit, the key-tile kernels otherwise.
        return hip_ops.attention_gradients(q, k, v, scales, out, grad, causal)

    def recompute():
        with torch.enable_grad():
            ins = [t.detach().requires_grad_() for t in (q, k, v, scales)]
            ref = routed_attention_reference(*ins, causal)
            return torch.autograd.grad(ref, ins, grad)

    def timed(fn, reps):
        for _ in range(max(args.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    # One SharedDictionaryAttention training step (forward + backward) on the
    # HIP backend beside the same module on the bf16 torch backend.
    torch.manual_seed(0)
    hip_module = da.SharedDictionaryAttention(config).to(device, torch.bfloat16)
    torch_module = da.SharedDictionaryAttention(config.with_updates(backend="torch")).to(device, torch.bfloat16)
    torch_module.load_state_dict(hip_module.state_dict())
    x = torch.randn(batch, length, d, generator=g).to(device, torch.bfloat16).requires_grad_()
    grad_x = torch.randn(batch, length, d, generator=g).to(device, torch.bfloat16)

    def train_step(m):
        def run():
            # A fresh step each rep: no gradient accumulation into .grad.
            x.grad = None
            for param in m.parameters():
                param.grad = None
            m(x).backward(grad_x)
        return run

    if args.kernels_only:
        # Only the HIP training step (and for C4 the HIP LM step), for a
        # kernel trace of what one step launches: args.steps reps, no timing.
        step = train_step(hip_module)
        for _ in range(args.steps):
            step()
        if args.workload == "c4":
            kwargs = dict(dictionary_group_size=LM_LAYERS, feedforward_dim=LM_FEEDFORWARD)
            lm = da.DoubleAttentionLM(LM_VOCAB, length, config, LM_LAYERS, **kwargs).to(device, torch.bfloat16)
            ids = torch.randint(0, LM_VOCAB, (batch, length), generator=g).to(device)
            targets = torch.randint(0, LM_VOCAB, (batch, length), generator=g).to(device)
            for _ in range(args.steps):
                for param in lm.parameters():
                    param.grad = None
                lm(ids, targets)[1].backward()
        torch.cuda.synchronize()
        print(json.dumps({"workload": args.workload, "training_steps": args.steps}), flush=True)
        return
    module_ms = {name: round(timed(train_step(m), max(1, min(args.steps, 20))), 4)
                 for name, m in (("hip", hip_module), ("torch_bf16", torch_module))}
    del hip_module, torch_module
    lm_ms = None
    if args.workload == "c4":
        # The LM training step (token ids to loss, then backward) on both
        # backends: the counterpart of the reference's LM fwd+bwd benchmark.
        kwargs = dict(dictionary_group_size=LM_LAYERS, feedforward_dim=LM_FEEDFORWARD)
        hip_lm = da.DoubleAttentionLM(LM_VOCAB, length, config, LM_LAYERS, **kwargs).to(device, torch.bfloat16)
        torch_lm = da.DoubleAttentionLM(
            LM_VOCAB, length, config.with_updates(backend="torch"), LM_LAYERS, **kwargs
        ).to(device, torch.bfloat16)
        torch_lm.load_state_dict(hip_lm.state_dict())
        ids = torch.randint(0, LM_VOCAB, (batch, length), generator=g).to(device)
        targets = torch.randint(0, LM_VOCAB, (batch, length), generator=g).to(device)

        def lm_step(m):
            def run():
                for param in m.parameters():
                    param.grad = None
                m(ids, targets)[1].backward()
            return run

        lm_ms = {name: round(timed(lm_step(m), max(1, min(args.steps, 20))), 4)
                 for name, m in (("hip", hip_lm), ("torch_bf16", torch_lm))}
        del hip_lm, torch_lm

    if not hip_ops._native_backward_supported(q, v):
        print(json.dumps({
            "metric": "outer-attention backward (dQ, dK, dV, dscale) on 1 MI355X",
            "value": None, "unit": "TFLOP/s",
            "note": f"score width {rp} has no native backward (widths up to 512); autograd recomputes in torch",
            "module_fwd_bwd_ms": module_ms,
            "config": {"workload": description, "score_dim": rp},
        }), flush=True)
        return
    ms = timed(native, args.steps)
    ref_ms = timed(recompute, max(1, min(args.steps, 20))) if length <= 4096 else None
    flops = 2.0 * batch * S * length * length * (4 * rp + 2 * d) * (0.5 if causal else 1.0)
    print(json.dumps({
        "metric": "outer-attention backward (dQ, dK, dV, dscale) on 1 MI355X",
        "value": round(flops / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "steps": args.steps,
        "torch_recompute_ms": None if ref_ms is None else round(ref_ms, 4),
        "speedup_vs_recompute": None if ref_ms is None else round(ref_ms / ms, 2),
        "module_fwd_bwd_ms": module_ms,
        "lm_fwd_bwd_ms": lm_ms,
        "attention_backward_path": "dense" if hip_ops._dense_backward_fits(q, v) else "key-tile kernels",
        "dtype": "fp16 q/k, bf16 v",
        "config": {"workload": description, "batch": batch, "maps": S, "length": length, "score_dim": rp,
                   "value_dim": d, "causal": causal},
    }), flush=True)


def compare_library() -> None:
    """GEMMs at the C1-C5 shapes: the library's hand GEMM (with its fused
    epilogues: V^T layout and bias for the Q/K/V projection, GELU, residual)
    against torch's GEMM (hipBLASLt) with the same epilogue as separate ops
    and without it; every launch replayed 20 at a time from a HIP graph, so
    host work is not timed.  Then the C1-C5 forwards (C4: the six-layer LM)
    on backend="hip" against backend="torch" in bf16 on the same GPU, eager,
    HIP events over 30 forwards (best of three), the reference's own forward
    comparison (Triton against its PyTorch path)."""

    import torch
    import torch.nn.functional as F

    import double_attention as da
    from double_attention import hip_ops

    dev = torch.device("cuda:0")

    def graph_us(fn, calls=20, replays=20):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(calls):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(replays):
                graph.replay()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3 / (replays * calls))
        return round(best, 2)

    def eager_us(fn, reps=30):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3 / reps)
        return round(best, 2)

    gen = torch.Generator().manual_seed(0)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=gen) * scale).to(dev, torch.bfloat16)

    gemms = []
    for name, (batch, length, width) in {"c1": (8, 512, 256), "c2": (8, 1024, 512), "c3": (4, 2048, 512),
                                         "c4": (64, 64, 512), "c5": (1, 8192, 256)}.items():
        x = rnd(batch, length, 512)
        wq, wk, wv = (rnd(n, 512, scale=512 ** -0.5) for n in (width, width, 512))
        bv = rnd(512)
        wcat = torch.cat([wq, wk, wv])
        bcat = torch.cat([torch.zeros(2 * width, dtype=bv.dtype, device=dev), bv])
        gemms.append({
            "gemm": f"{name} Q/K/V projection {batch * length}x512 -> {2 * width}+512",
            "hip_us": graph_us(lambda: hip_ops.qkv_projection_hip(x, wq, wk, wv, bv)),
            "torch_us": graph_us(lambda: F.linear(x, wcat, bcat)),
            "gflop": round(2 * batch * length * 512 * (2 * width + 512) / 1e9, 3),
        })
    for name, (n, k, o, act, res) in {
        "c1 output projection": (4096, 512, 512, None, False),
        "c2/c3/c5 output projection": (8192, 512, 512, None, False),
        "c4 output projection + residual": (4096, 512, 512, None, True),
        "c4 FFN up + bias + GELU": (4096, 512, 1536, "gelu", False),
        "c4 FFN down + bias + residual": (4096, 1536, 512, None, True),
    }.items():
        x = rnd(n, k)
        w = rnd(o, k, scale=k ** -0.5)
        bias = rnd(o) if (act or res) else None
        r = rnd(n, o) if res else None
        if act == "gelu":
            unfused = lambda: F.gelu(F.linear(x, w, bias))  # noqa: E731
        elif res:
            unfused = lambda: r + F.linear(x, w, bias)  # noqa: E731
        else:
            unfused = lambda: F.linear(x, w)  # noqa: E731
        gemms.append({
            "gemm": f"{name} {n}x{k} -> {o}",
            "hip_us": graph_us(lambda: hip_ops.linear_hip(x, w, bias, activation=act, residual=r)),
            "torch_us": graph_us(unfused),
            "torch_gemm_only_us": graph_us(lambda: F.linear(x, w, bias)),
            "gflop": round(2 * n * k * o / 1e9, 3),
        })
    forwards = []
    for name in ("c1", "c2", "c3", "c5", "c4"):
        preset, batch, length, overrides, _ = WORKLOADS[name]
        config = da.experiment_config(preset, backend="hip", **overrides)
        torch.manual_seed(0)
        if name == "c4":
            hip = da.DoubleAttentionLM(LM_VOCAB, length, config, LM_LAYERS, dictionary_group_size=LM_LAYERS,
                                       feedforward_dim=LM_FEEDFORWARD).to(dev, torch.bfloat16).eval()
            ref = da.DoubleAttentionLM(LM_VOCAB, length, config.with_updates(backend="torch"), LM_LAYERS,
                                       dictionary_group_size=LM_LAYERS,
                                       feedforward_dim=LM_FEEDFORWARD).to(dev, torch.bfloat16).eval()
            inp = torch.randint(0, LM_VOCAB, (batch, length), generator=torch.Generator().manual_seed(1)).to(dev)
        else:
            hip = da.SharedDictionaryAttention(config).to(dev, torch.bfloat16).eval()
            ref = da.SharedDictionaryAttention(config.with_updates(backend="torch")).to(dev, torch.bfloat16).eval()
            inp = torch.randn(batch, length, config.model_dim, generator=torch.Generator().manual_seed(1)).to(
                dev, torch.bfloat16)
        ref.load_state_dict(hip.state_dict())
        with torch.inference_mode():
            t_hip, t_ref = eager_us(lambda: hip(inp)), eager_us(lambda: ref(inp))
        forwards.append({"workload": name, "hip_us": t_hip, "torch_bf16_us": t_ref,
                         "speedup": round(t_ref / t_hip, 2)})
        del hip, ref
    print(json.dumps({"compare_library": {"gemms": gemms, "forwards": forwards}}), flush=True)


def main() -> None:
    args = parse_args()
    if args.collect_counters:
        collect_counters(args)
        return
    if args.compare_library and args.gpus == 1:
        compare_library()
        return
    if args.backward and args.gpus == 1:
        backward_bench(args)
        calibration_copy(args.copy_mib, "cuda:0")
        return
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only: this build has no multi-GPU path "
            f"(requested --gpus {args.gpus}); run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    import double_attention as da
    from double_attention import _lib

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    lib = _lib.get()
    device = torch.device("cuda:0")
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    code = _lib.DA_BF16 if dtype == torch.bfloat16 else _lib.DA_F16
    preset, batch, length, overrides, description = WORKLOADS[args.workload]
    config = da.experiment_config(preset, backend="hip", **overrides)
    torch.manual_seed(0)
    lm = None
    if args.workload == "c4":
        lm = da.DoubleAttentionLM(
            LM_VOCAB, length, config, LM_LAYERS, dictionary_group_size=LM_LAYERS, feedforward_dim=LM_FEEDFORWARD
        ).to(device=device, dtype=dtype).eval()
        ids = torch.randint(0, LM_VOCAB, (batch, length), generator=torch.Generator().manual_seed(1)).to(device)
        module = lm.stack.blocks[0].attention
        bank = lm.stack.banks[0]

        def step():
            return lm(ids)[0]
    else:
        module = da.SharedDictionaryAttention(config).to(device=device, dtype=dtype).eval()
        bank = module.bank

        def step():
            return module(x)

    # The attention input (for C4: one layer's, the LayerNorm output's shape).
    x = torch.randn(batch, length, config.model_dim, generator=torch.Generator().manual_seed(1)).to(device, dtype)

    # ---- whole forward (the step) ----------------------------------------
    torch.cuda.reset_peak_memory_stats(device)
    timed_steps = 0 if args.kernels_only else args.steps
    with torch.inference_mode():
        for _ in range(args.warmup if timed_steps else 0):
            step()
        torch.cuda.synchronize()
        start = time.perf_counter()
        out = None
        for _ in range(timed_steps):
            out = step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start
    ms_per_step = elapsed * 1e3 / max(timed_steps, 1)
    # Peak device memory of the step loop (the reference's harness reports
    # max_memory_allocated beside its timings): weights, input, workspace, outputs.
    peak_mib = torch.cuda.max_memory_allocated(device) / 2**20
    graph_ms = None
    if lm is not None and timed_steps:
        # The same LM forward replayed as one HIP graph (no per-call host work).
        graphed = da.GraphedForward(lm, ids)
        for _ in range(args.warmup):
            graphed(ids)
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(args.steps):
            graphed(ids)
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - start) * 1e3 / args.steps
        del graphed
    tokens = batch * length
    H, S, R, M, d = config.qk_branches, config.outer_maps, config.routing_dim, config.dictionary_size, config.model_dim
    W = H * R
    rows = 2 * batch * H * length
    group = H // S if H > S else 1
    rp = group * R

    # ---- per-kernel timing on the launch stream ---------------------------
    stream = torch.cuda.current_stream(device)
    handle = stream.cuda_stream
    with torch.inference_mode():
        key_dtype = da.hip_ops.route_key_dtype(config.normalize_routing_input, dtype)
        key_code = da.hip_ops.dtype_code(key_dtype)
        key, value = bank.normalized_hip(config.eps, key_dtype)
        layout = key._da_route_layout
        qk = torch.empty(tokens, 2 * W, device=device, dtype=dtype)
        tp = lib.da_padded_length(length)
        vt = torch.zeros(batch, tp // 32, d, 32, device=device, dtype=dtype)
        routed = torch.empty(tokens, 2 * W, device=device, dtype=torch.float16)
        mixed = torch.empty(tokens, d, device=device, dtype=dtype)
        final = torch.empty(tokens, d, device=device, dtype=dtype)
        p = {k: v.contiguous() for k, v in module.state_dict().items()}
        pdt = da.hip_ops.dtype_code(p["log_beta"].dtype)
        raw_key = bank.raw_key.detach()
        raw_value = bank.raw_value.detach() if bank.raw_value is not None else None

        variant = da.hip_ops.RouteVariant.of_config(config)
        route_flags = (
            _lib.DA_ROUTE_BETA_IS_LOG | _lib.DA_ROUTE_UNIT_KEYS | variant.flags()
            | (_lib.DA_ROUTE_NORMALIZE_INPUT if config.normalize_routing_input else 0)
            | (_lib.DA_ROUTE_NORMALIZE_OUTPUT if config.normalize_routing_output else 0)
        )
        attn_flags = _lib.DA_ATTN_CAUSAL | _lib.DA_ATTN_SCALES_ARE_LOG | _lib.DA_ATTN_MIX
        attn_ws_bytes = lib.da_attention_workspace_bytes(batch, S, length, rp, d, attn_flags)
        attn_ws = torch.empty(attn_ws_bytes, dtype=torch.uint8, device=device) if attn_ws_bytes else None
        launches = {
            "dict_normalize": lambda: lib.da_dictionary_normalize(
                raw_key.data_ptr(), None if raw_value is None else raw_value.data_ptr(),
                da.hip_ops.dtype_code(raw_key.dtype), R, M, config.eps,
                layout.key_t.data_ptr(), key_code, layout.value.data_ptr(), None, handle),
            "qkv_projection": lambda: lib.da_qkv_projection(
                x.data_ptr(), tokens, d, length, p["query.weight"].data_ptr(), p["key.weight"].data_ptr(), W,
                p["value.weight"].data_ptr(), p["value.bias"].data_ptr(), d, pdt, code,
                qk.data_ptr(), vt.data_ptr(), vt.stride(0), tp, handle),
            "route": lambda: lib.da_dictionary_route(
                qk.data_ptr(), rows, R, R, code, layout.key_t.data_ptr(), key_code, layout.value.data_ptr(), M,
                p["log_beta"].data_ptr(), pdt, 0.0, config.eps, route_flags, variant.silu_gain,
                variant.logit_scale(R), routed.data_ptr(), R, _lib.DA_F16, handle),
            "attention": lambda: lib.da_routed_attention(
                routed.data_ptr(), routed.data_ptr() + W * routed.element_size(), length * 2 * W, 2 * W,
                rp if H > S else R, S // H if S > H else 1, rp, vt.data_ptr(), vt.stride(0),
                batch, S, length, d, p["log_score_scales"].data_ptr(), pdt,
                float(group ** -0.5), None if S == 1 else p["map_mix_logits"].data_ptr(), pdt,
                _lib.DA_ATTN_CAUSAL | _lib.DA_ATTN_SCALES_ARE_LOG | _lib.DA_ATTN_MIX,
                1.01 * group if config.normalize_routing_output else 0.0, _lib.DA_F16, code,
                mixed.data_ptr(), length * d, d, 0,
                attn_ws.data_ptr() if attn_ws is not None else None, attn_ws_bytes, handle),
            "output_projection": lambda: lib.da_linear(
                mixed.data_ptr(), tokens, d, p["output.weight"].data_ptr(), d, None, pdt, code,
                final.data_ptr(), handle),
        }
        kernel_us = {}
        for name, launch in launches.items():
            for _ in range(5):
                _lib.check(launch(), name)
            torch.cuda.synchronize()
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            begin.record(stream)
            for _ in range(args.kernel_reps):
                launch()
            end.record(stream)
            end.synchronize()
            kernel_us[name] = begin.elapsed_time(end) * 1e3 / args.kernel_reps
        # The memory-bound stages once more, each launch alone after a 512 MiB
        # device write that evicts the 256 MB Infinity Cache and the L2s: the
        # back-to-back loop above reads operands a previous launch left in
        # cache.  Median of 20 launches.
        flush = torch.empty(512 << 20, dtype=torch.uint8, device=device)
        flushed_us = {}
        for name in () if args.kernels_only else ("dict_normalize", "qkv_projection", "output_projection"):
            samples = []
            for _ in range(20):
                flush.fill_(1)
                begin = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                begin.record(stream)
                launches[name]()
                end.record(stream)
                end.synchronize()
                samples.append(begin.elapsed_time(end) * 1e3)
            flushed_us[name] = sorted(samples)[len(samples) // 2]
        del flush
    if args.kernels_only:
        print(json.dumps({"workload": args.workload, "kernel_order": list(launches), "kernel_us": kernel_us}), flush=True)
        calibration_copy(args.copy_mib, device)
        return

    flops = {
        "route": 4.0 * R * M * rows,
        "attention": 2.0 * (rp + d) * length * (length + 1) / 2 * batch * S,
        "qkv_projection": 2.0 * tokens * d * (2 * W + d),
        "output_projection": 2.0 * tokens * d * d,
    }
    elem = 2
    n_dict = 1 if raw_value is None else 2
    in_elem = raw_key.element_size()
    bytes_moved = {
        "dict_normalize": n_dict * R * M * in_elem + 2 * R * M * elem,
        "qkv_projection": (tokens * d + (2 * W + d) * d + tokens * (2 * W + d)) * elem,
        "output_projection": (2 * tokens * d + d * d) * elem,
    }
    dominant = max(("route", "attention", "qkv_projection", "output_projection"), key=lambda k: kernel_us[k])
    achieved = flops[dominant] / (kernel_us[dominant] * 1e-6) / 1e12
    roofline = {
        "kernel": dominant,
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "traffic": None,
        "avg_launch_us": round(kernel_us[dominant], 3),
    }
    # Counter evidence for the same kernel sources (--collect-counters):
    # rocprofv3's MFMA-busy fraction beside the algorithmic one, the MFMA
    # flops the kernel executed, and HBM bytes per launch.
    counters = measured_counters(args.workload)
    if counters is not None and dominant in counters["kernels"]:
        c = counters["kernels"][dominant]
        roofline["traffic"] = c.get("hbm_bytes_per_launch")
        roofline["counter_mfma_busy"] = c.get("mfma_busy")
        if c.get("mfma_flops_executed"):
            roofline["counter_mfma_flops_executed"] = c["mfma_flops_executed"]
            roofline["algorithmic_flops"] = flops[dominant]
        roofline["counters"] = f"profiles/counters_{args.workload}.json"
    kernels = {}
    for name, us in kernel_us.items():
        entry = {"avg_us": round(us, 3)}
        if name in flops:
            tf = flops[name] / (us * 1e-6) / 1e12
            entry.update(tflops=round(tf, 2), mfma_frac=round(tf / PEAK_BF16_TFLOPS, 4))
        if name in bytes_moved:
            gbs = bytes_moved[name] / (us * 1e-6) / 1e9
            entry.update(gbs=round(gbs, 1), hbm_frac=round(gbs / PEAK_HBM_GBS, 4))
        if counters is not None and name in counters["kernels"]:
            c = counters["kernels"][name]
            entry.update({k: c[k] for k in ("mfma_busy", "hbm_bytes_per_launch") if k in c})
        if name in flushed_us:
            fus = flushed_us[name]
            fgbs = bytes_moved[name] / (fus * 1e-6) / 1e9
            entry.update(flushed_us=round(fus, 3), flushed_gbs=round(fgbs, 1),
                         flushed_hbm_frac=round(fgbs / PEAK_HBM_GBS, 4))
        kernels[name] = entry

    # ---- CPU baseline: this package's backend="torch" fp32 path -----------
    # The same seeded weights and input, on the host's cores: inference
    # mode, two warmups, then the median of at least five forwards (three
    # for the long-context C5, whose torch path materializes 8192^2 scores).
    cpu = None
    if not args.no_cpu_baseline:
        import statistics

        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        host = cpu_info()
        cpu_config = config.with_updates(backend="torch")
        if lm is not None:
            cpu_model_ = da.DoubleAttentionLM(
                LM_VOCAB, length, cpu_config, LM_LAYERS, dictionary_group_size=LM_LAYERS,
                feedforward_dim=LM_FEEDFORWARD,
            ).eval()
            cpu_model_.load_state_dict({k: v.float().cpu() for k, v in lm.state_dict().items()})
            cpu_in = ids.cpu()

            def cpu_step():
                return cpu_model_(cpu_in)[0]
        else:
            cpu_model_ = da.SharedDictionaryAttention(cpu_config).eval()
            cpu_model_.load_state_dict({k: v.float().cpu() for k, v in module.state_dict().items()})
            cpu_in = x.float().cpu()

            def cpu_step():
                return cpu_model_(cpu_in)
        reps = 3 if args.workload == "c5" else 5
        times = []
        with torch.inference_mode():
            for _ in range(2):
                cpu_step()
            for _ in range(reps):
                t0 = time.perf_counter()
                cpu_step()
                times.append(time.perf_counter() - t0)
        cpu_ms = statistics.median(times) * 1e3
        cpu = {
            "value": round(tokens / (cpu_ms * 1e-3), 1),
            "unit": "tokens/s",
            "ms_per_step": round(cpu_ms, 2),
            "routed_rows_per_s": round(rows / (cpu_ms * 1e-3), 1),
            "cores": threads,
            "kind": "port",
            "host": host,
            "sample": f"median of {reps} {args.workload} forwards (after 2 warmups) of this package's backend='torch' "
                      f"fp32 module on {threads} threads ({host['model']}, {host['physical_cores']} physical cores, "
                      f"{host['threads']} threads), same weights and input",
        }
        del cpu_model_

    line = {
        "metric": METRIC,
        "value": round(tokens / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic: x ~ N(0,1) seeded, default-init weights seeded",
        "config": {
            "workload": description,
            "preset": preset,
            "global_batch": batch,
            "seq_len": length,
            "routed_rows": rows,
            **({"layers": LM_LAYERS, "vocab": LM_VOCAB, "feedforward_dim": LM_FEEDFORWARD} if lm is not None else {}),
            "parallelism": "single GPU",
        },
        "routed_rows_per_s": round(rows / (kernel_us["route"] * 1e-6), 1),
        "attention_tokens_per_s": round(tokens / (kernel_us["attention"] * 1e-6), 1),
        **({"graph_ms_per_step": round(graph_ms, 4)} if graph_ms is not None else {}),
        "peak_memory_mib": round(peak_mib, 1),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    del out

    calibration_copy(args.copy_mib, device)


def calibration_copy(mib: int, device) -> None:
    """Copy a device buffer of ``mib`` MiB three times: a kernel of known
    traffic that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""

    import torch

    if mib <= 0:
        return
    src = torch.empty(mib << 20, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


if __name__ == "__main__":
    main()
