#!/usr/bin/env python3
"""Benchmark of the MI355X decode/prefill path (BASELINE config 2 by default).

Workload (one GPU): the Qwen3.5-0.8B-shaped hybrid with random-init fp32
weights (N(0, 0.02), seed 0), a 454-token uniform random prompt (seed 4),
greedy decode. A step is one decode forward (one token) including the device
argmax readback, as the reference times `step_greedy` (src/device/cli.rs:797-812).
`--warmup` untimed steps, then exactly `--steps` timed steps bracketed by a
stream synchronisation on both sides. value = decode tokens/s at ctx 454.

Also reported: weight-read HBM GB/s of the decode step; the prefill rate of
the prompt; the 2644- and 10,240-token prefills (config 3: median of timed
runs, tok/s, the fp32-equivalent FLOP rate, the BF16 part products it
executes and the fraction of the prefill time the work would take at the
peaks of the instructions executed; --no-prefill skips); the 4-row verify
and speculative generation (n-gram and known-continuation drafts) against
plain greedy (--no-spec skips); decode at ctx 8192 after a real 8192-token
prefill (config 4; --no-long skips); int8 decode at ctx 454, its 4-row
verify with snapshots and speculative rates (config 5; --no-int8 skips);
BF16 decode at ctx 454 on the BF16-rounded weights (--no-bf16 skips);
the drop-in rates (an unmodified reference engine: the op
sequence of bridge calls, no one-launch step or fp32 fusions, prefill in
128-token chunks; --no-dropin skips). roofline: the one-launch decode kernel
(decode_kernel: every layer, lm_head and argmax of a step), timed with a
hipEvent pair around each launch on the bridge's stream in a profiled pass of
the same decode; achieved = the step's algorithmic HBM bytes (every matrix
once, DeltaNet recurrent and conv states read and written, K/V rows of the
context read and the new row written, logits written) / launch duration.
cpu_baseline: the CPU oracle (restatement of the reference's Backend::Vector
path) on this host: decode steps at ctx 454 from the GPU run's state after
the prompt (the value), and token-by-token prefill steps near ctx 2644; one
warmup step, then --cpu-runs runs of --cpu-steps steps each, at the
reference's default thread count min(cores, 8) and at every core of this
job's CPU share (at most 16 on a one-GPU box).
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "qwen-rust-inference_amd"), str(ROOT / "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
# HBM bytes per decode_kernel launch at ctx ~475 from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
# (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0, calibrated on a 512 MiB copy; profiles/decode_kernel_config2.md).
DECODE_TRAFFIC_BYTES = 3_154_785_217
PREFILL_CHUNK = 128  # the reference engine's prefill chunk (src/device.rs)


def mall_resident_bytes(c) -> int:
    """Weight bytes the one-launch decode reads with allocating loads below
    position 1536 (csrc/decode.hip kKeepAqkv / kKeepDin, fp32): part 0 (rows
    3u and 3u + 1) of q|k|v in every attention layer and part 0 (rows 4u and
    4u + 1) of qkv|a|b in the DeltaNet layers among layers 0-11, over the
    2048 wave units u. They stay in the 256 MB memory-side cache between
    steps, so that part of the weight-read rate is not HBM traffic."""
    units = 2048
    aqkv_rows = 2 * c.num_heads * c.head_dim + 2 * c.num_kv_heads * c.head_dim
    din_rows = c.channels + 2 * c.value_heads
    aqkv = sum(1 for u in range(units) for r in (0, 1) if 3 * u + r < aqkv_rows)
    din = sum(1 for u in range(units) for r in (0, 1) if 4 * u + r < din_rows)
    row = 4 * c.hidden_size
    attn = [layer for layer in range(c.num_layers) if c.attention[layer]]
    delta_kept = [layer for layer in range(min(12, c.num_layers)) if not c.attention[layer]]
    return row * (aqkv * len(attn) + din * len(delta_kept))


def host_cpu():
    """nproc, the CPU model and the cgroup CPU quota (the reference records the
    same, src/benchmark.rs:156-174)."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        quota = open("/sys/fs/cgroup/cpu.max").read().strip()
    except OSError:
        quota = "n/a"
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "model": model, "cgroup_cpu_max": quota}


MFMA_F32_PEAK_TFLOPS = 157.3
METRIC = "decode tok/s @ctx 454 & 8192 + HBM GB/s; prefill tok/s @2644"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(label: str) -> int:
    """Weight bytes one profiled fp32 GEMV call reads, from its label
    ("gemv_f32 248320x1024", "gemv_f32_group 6144x1024+2048x1024", "..._glu 2x3584x1024")."""
    body = label.split(" ", 1)[1].split(" t")[0]
    total = 0
    mult = 1
    if body.startswith("2x"):
        mult, body = 2, body[2:]
    for part in body.split("+"):
        r, c = part.split("x")
        total += int(r) * int(c) * 4
    return total * mult


def step_bytes(c, weight_bytes: int, length: int) -> int:
    """Algorithmic HBM bytes of one decode step whose token sits at position
    length - 1: every matrix once (lm_head = the tied embedding), the DeltaNet
    recurrent and conv states read and written, length - 1 cached K/V rows
    read and one written, the logits written."""
    attn = sum(1 for a in c.attention[:c.num_layers] if a)
    delta = c.num_layers - attn
    recurrent = c.value_heads * c.key_dim * c.value_dim * 4
    conv = c.channels * (c.conv_kernel - 1) * 4
    kv_row = 2 * c.num_kv_heads * c.head_dim * 4
    return (weight_bytes + delta * 2 * (recurrent + conv) + attn * length * kv_row + c.vocab_size * 4)


def prefill_flops(c, n: int, weight_params: int) -> float:
    """Algorithmic FLOPs of an n-token prefill: every projection but lm_head
    on n rows, lm_head on the last row, causal attention (QK^T and PV,
    n(n+1)/2 pairs per head), and the chunked DeltaRule (per chunk and head:
    the Gram products, the triangular solve, U / W, and the three scan
    products)."""
    return sum(prefill_flop_parts(c, n, weight_params))


def prefill_flop_parts(c, n: int, weight_params: int):
    """(projections, attention, DeltaRule) FLOPs of prefill_flops."""
    vocab_params = c.vocab_size * c.hidden_size
    proj = 2.0 * (weight_params - vocab_params) * n + 2.0 * vocab_params
    attn_layers = sum(1 for t in c.layer_types if t == "full_attention")
    attn = attn_layers * c.num_heads * 4.0 * c.head_dim * n * (n + 1) / 2
    dk, dv, ch = c.key_dim, c.value_dim, 64
    per_chunk = 2.0 * (2 * ch * ch * dk + ch * ch * (dk + dv) / 2 + 2 * ch * dk * dv + ch * ch * dv + dk * ch * dv)
    rule = (len(c.layer_types) - attn_layers) * c.value_heads * -(-n // ch) * per_chunk
    return proj, attn, rule


# Part products per fp32 multiply-add on the BF16 MFMA (x = x0 + x1 + x2 for
# both operands, the six products with p + q <= 2): the prefill projections
# (csrc/gemm_p3.hip) and prefill attention (attention_prefill_bf3_kernel) run
# on v_mfma_f32_32x32x16_bf16 at this multiple of the fp32-equivalent FLOPs;
# the chunked DeltaRule runs on fp32 MFMA (v_mfma_f32_16x16x4_f32).
BF16_PARTS = 6
MFMA_BF16_PEAK_TFLOPS = 2500.0


class KnownDraft:
    """A draft that proposes the true greedy continuation (known from a plain
    greedy run of the same model): every drafted token is accepted, so a
    speculative pass of depth k emits k + 1 tokens. The upper bound of what
    the one-pass verify gives a draft model."""

    def __init__(self, prompt, continuation):
        self.seq = list(prompt[1:]) + list(continuation)
        self.n = 0

    def absorb(self, tokens):
        self.n += len(tokens)

    def draft(self, k):
        return self.seq[self.n:self.n + k]


def speculative_rates(E, model, prompt, depth: int, n_new: int, snapshots: int):
    """Plain greedy and speculative (n-gram and known-continuation drafts)
    generation of n_new tokens after `prompt` on fresh runs: tok/s of the
    decode part (prefill excluded), the verify pass cost and acceptance."""
    out = {}
    r = model.new_run(len(prompt) + n_new + 8, chunk=len(prompt), snapshots=snapshots)
    tok = int(__import__("numpy").argmax(r.prefill(prompt)))
    model.sync()
    ids, _ = r.decode_greedy(tok, 2)  # warm
    r.close()
    r = model.new_run(len(prompt) + n_new + 8, chunk=len(prompt), snapshots=snapshots)
    tok = int(__import__("numpy").argmax(r.prefill(prompt)))
    model.sync()
    t = time.perf_counter()
    ids, _ = r.decode_greedy(tok, n_new)
    model.sync()
    out["greedy_tok_s"] = round((n_new - 1) / (time.perf_counter() - t), 1)
    r.close()
    for name, draft in (("ngram", "ngram"), ("known", KnownDraft(prompt, ids))):
        for rep in range(2):  # the first pass warms the verify code path
            if name == "known":
                draft.n = 0
            r = model.new_run(len(prompt) + n_new + 8, chunk=len(prompt), snapshots=snapshots)
            model.sync()
            t = time.perf_counter()
            got, st = r.speculative_generate(prompt, n_new, depth, draft=draft)
            model.sync()
            wall = time.perf_counter() - t
            r.close()
        same = got == ids
        out[name] = {"tok_s": round((len(got) - 1) / (wall - st["prefill_s"]), 1), "passes": st["passes"],
                     "accepted": st["accepted"], "offered": st["offered"], "equals_greedy": same}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prompt", type=int, default=454)
    ap.add_argument("--no-prefill", dest="prefill", action="store_false",
                    help="skip the 2644- and 10,240-token prefills (config 3)")
    ap.add_argument("--no-long", dest="long", action="store_false", help="skip decode at ctx 8192 (config 4)")
    ap.add_argument("--no-int8", dest="int8", action="store_false",
                    help="skip the int8 decode and 4-row verify at ctx 454 (config 5)")
    ap.add_argument("--no-spec", dest="spec", action="store_false",
                    help="skip the speculative-generation rates (fp32, and int8 with config 5)")
    ap.add_argument("--no-bf16", dest="bf16", action="store_false",
                    help="skip the BF16 decode (the model's weights rounded to BF16, every matrix uploaded as BF16)")
    ap.add_argument("--no-dropin", dest="dropin", action="store_false",
                    help="skip the drop-in (unmodified reference engine call sequence) rates")
    ap.add_argument("--cpu-steps", type=int, default=4,
                    help="timed oracle steps per run of the CPU baseline (0: skip)")
    ap.add_argument("--cpu-runs", type=int, default=2, help="timed runs per CPU baseline measurement")
    ap.add_argument("--profile-steps", type=int, default=16)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run one device copy of MIB MiB (a plain copy kernel of known size, the scale "
                         "for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--only-prefill", type=int, default=0, metavar="N",
                    help="profiling mode: only two N-token prefills (one chunk, fresh runs) and a one-line summary")
    ap.add_argument("--prefill-format", choices=["f32", "bf16", "int8"], default="f32",
                    help="with --only-prefill: the matrices' format (BF16: every tensor rounded to BF16)")
    args = ap.parse_args()
    if args.profile_steps < 1:
        ap.error("--profile-steps must be at least 1 (the roofline's per-launch time comes from them)")
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path's sharding is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import __graft_entry__
    if not __graft_entry__._built():
        __graft_entry__.build()
    from qwen_mi355x import engine as E
    from qwen_mi355x import model as M

    c = M.config_qwen08b(max_positions=16384)
    t0 = time.time()
    w = M.synthetic_weights(c, seed=0)
    log(f"weights synthesised in {time.time() - t0:.1f} s ({w.matrix_bytes() / 1e9:.3f} GB of matrices)")
    if args.only_prefill > 0 and args.prefill_format != "f32":
        model = E.Model(M.bf16_weights(w), fmt=E.BF16_EXACT) if args.prefill_format == "bf16" else E.Model(w, fmt=E.INT8)
    else:
        model = E.Model(w)
    log(model.info)
    model.set_run_budget(64 << 30)
    weight_bytes = w.matrix_bytes()
    if args.only_prefill > 0:
        n = args.only_prefill
        ids2 = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, n)]
        times = []
        for rep in range(2):
            r2 = model.new_run(n + 1, chunk=n)
            model.sync()
            t = time.perf_counter()
            r2.prefill(ids2)
            times.append(time.perf_counter() - t)
            r2.close()
        print(json.dumps({"mode": "only-prefill", "format": args.prefill_format, "tokens": n,
                          "prefill_ms": [round(x * 1e3, 2) for x in times]}), flush=True)
        model.close()
        return
    prompt = [int(v) for v in np.random.default_rng(4).integers(0, c.vocab_size, args.prompt)]

    # prefill of the prompt (one chunk), then decode; one untimed prefill of the
    # same length first (code objects, and the bridge's per-shape GEMM choice)
    cap = args.prompt + args.warmup + args.steps + args.profile_steps + 4
    warm = model.new_run(cap, chunk=args.prompt)
    warm.prefill(prompt)
    warm.close()
    run = model.new_run(cap, chunk=args.prompt)
    model.sync()
    t = time.perf_counter()
    logits = run.prefill(prompt)
    prefill_s = time.perf_counter() - t
    token = int(np.argmax(logits))
    log(f"prefill {args.prompt} tokens: {prefill_s * 1e3:.1f} ms")
    for _ in range(args.warmup):
        token = run.step_greedy(token)
    model.sync()
    t = time.perf_counter()
    ids, _ = run.decode_greedy(token, args.steps + 1)
    model.sync()
    decode_s = time.perf_counter() - t
    token = ids[-1]
    value = args.steps / decode_s
    ms = decode_s / args.steps * 1e3
    hbm = weight_bytes * value / 1e9
    log(f"one-launch decode plan: {run.decode_plan}")
    log(f"decode: {ms:.3f} ms/token, {value:.1f} tok/s, weight-read {hbm:.0f} GB/s ({hbm / HBM_PEAK_GBS:.1%} of peak)")

    # roofline pass: the same decode with the bridge's event profiler on
    pos0 = run.position
    model.profile(True)
    run.decode_greedy(token, args.profile_steps + 1)
    stats = model.profile_read()
    model.profile(False)
    total_ms = sum(v[1] for v in stats.values())
    for k, v in sorted(stats.items(), key=lambda kv: -kv[1][1])[:12]:
        log(f"  {v[1] / args.profile_steps * 1e3:9.1f} us/step {v[0] // args.profile_steps:4d} calls/step  {k}")
    if "decode_step" in stats:
        calls, step_ms = stats["decode_step"]
        bytes_total = sum(step_bytes(c, weight_bytes, p + 1) for p in range(pos0, pos0 + calls))
        achieved = bytes_total / (step_ms / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": DECODE_TRAFFIC_BYTES,
                    "kernel": "decode_kernel (one-launch decode step: 24 layers, lm_head, argmax)",
                    "bytes_per_launch": bytes_total // calls, "launch_us": round(step_ms / calls * 1e3, 2),
                    "mall_resident_bytes": mall_resident_bytes(c),
                    "note": "achieved counts every weight byte once per step; mall_resident_bytes of them are kept "
                            "in the 256 MB memory-side cache between steps and do not reach HBM",
                    "launches": calls, "context": [pos0 + 1, pos0 + calls],
                    "bridge_gpu_us_per_step": round(total_ms / args.profile_steps * 1e3, 1)}
    else:  # op sequence (the bridge declined the plan): the fp32 GEMVs
        gemv = {k: v for k, v in stats.items() if k.startswith("gemv_f32")}
        gemv_bytes_total = sum(gemv_bytes(k) * v[0] for k, v in gemv.items())
        gemv_ms = sum(v[1] for v in gemv.values())
        launches = sum(v[0] for v in gemv.values())
        achieved = gemv_bytes_total / (gemv_ms / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                    "kernel": "fp32 decode GEMV (gemv_kernel<F32,...>: every projection of a step, lm_head included)",
                    "bytes_per_step": gemv_bytes_total // args.profile_steps,
                    "launches_per_step": launches // args.profile_steps,
                    "gemv_us_per_step": round(gemv_ms / args.profile_steps * 1e3, 1),
                    "bridge_gpu_us_per_step": round(total_ms / args.profile_steps * 1e3, 1)}

    out = {"metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": "config 2: Qwen3.5-0.8B-shaped hybrid, fp32 random-init weights, "
                                  f"{args.prompt}-token prompt, batch-1 greedy decode",
                      "prompt_tokens": args.prompt, "weights_seed": 0, "prompt_seed": 4,
                      "weight_bytes_per_token": weight_bytes},
           "hbm_weight_read_gbs": round(hbm, 1), "hbm_weight_read_frac": round(hbm / HBM_PEAK_GBS, 4),
           f"prefill_{args.prompt}_tok_s": round(args.prompt / prefill_s, 1),
           "roofline": roofline}

    # attainable read bandwidth: the stream-read program (4 GiB, the decode
    # kernel's load pattern) in a child process, median of 10 passes
    reader = ROOT / "qwen-rust-inference_amd" / "bin" / "stream_read"
    if reader.exists():
        import subprocess
        r = subprocess.run([str(reader), "4096", "10"], capture_output=True, text=True, timeout=120)
        if r.returncode == 0 and r.stdout.strip():
            sr = json.loads(r.stdout.strip().splitlines()[-1])
            out["hbm_stream_read_gbs"] = sr["gbs"]
            out["hbm_weight_read_frac_of_stream_read"] = round(hbm / sr["gbs"], 4)
            roofline["attainable"] = sr["gbs"]
            log(f"stream read: {sr['gbs']:.0f} GB/s attainable ({sr['gbs'] / HBM_PEAK_GBS:.1%} of the nominal peak); "
                f"decode weight-read is {hbm / sr['gbs']:.1%} of it")
        else:
            log(f"stream read failed: {r.stderr.strip()[-200:]}")

    def verify4_ms(m, fmt_prompt):
        """A 4-row verify with per-row snapshots + accept(1) (the rows' logits
        rolled back but the first), after one untimed pass."""
        rv = m.new_run(len(fmt_prompt) + 160, chunk=len(fmt_prompt), snapshots=3)
        tk = int(np.argmax(rv.prefill(fmt_prompt)))
        idv, _ = rv.decode_greedy(tk, 3)
        draft = [int(v) for v in np.random.default_rng(6).integers(0, c.vocab_size, 4)]
        rv.verify_rollback_greedy(draft)
        rv.accept(1)
        m.sync()
        reps = 16
        t0 = time.perf_counter()
        for _ in range(reps):
            rv.verify_rollback_greedy(draft)
            rv.accept(1)
        m.sync()
        dt = (time.perf_counter() - t0) / reps
        rv.close()
        return dt * 1e3

    if args.spec:
        # Speculative generation (the reference's generate loop, depth 3: one
        # 4-row verify pass per step) against plain greedy on the same model:
        # the engine's n-gram prompt-lookup draft, and a draft that knows the
        # greedy continuation (every token accepted: the one-pass verify's
        # upper bound for a real draft model).
        out["verify4_ms"] = round(verify4_ms(model, prompt), 3)
        spec = speculative_rates(E, model, prompt, 3, 64, 3)
        out["speculative_454"] = spec
        log(f"fp32 4-row verify + accept(1): {out['verify4_ms']:.3f} ms; speculative depth 3 over 64 tokens: "
            f"greedy {spec['greedy_tok_s']} tok/s, n-gram draft {spec['ngram']['tok_s']} tok/s "
            f"(accepted {spec['ngram']['accepted']}), known draft {spec['known']['tok_s']} tok/s")

    if args.long:
        # Decode at ctx 8192 (config 4): a real prefill of 8192 uniform random
        # ids (seed 5, one chunk), then 2 untimed and 64 timed greedy steps.
        n = 8192
        ids4 = [int(v) for v in np.random.default_rng(5).integers(0, c.vocab_size, n)]
        r3 = model.new_run(n + 80, chunk=n)
        tok = int(np.argmax(r3.prefill(ids4)))
        for _ in range(2):
            tok = r3.step_greedy(tok)
        model.sync()
        t = time.perf_counter()
        r3.decode_greedy(tok, 65)
        dt = time.perf_counter() - t
        long_bytes = sum(step_bytes(c, weight_bytes, p + 1) for p in range(n + 2, n + 66)) / 64
        out["decode_8192_tok_s"] = round(64 / dt, 2)
        out["decode_8192_hbm_frac"] = round(long_bytes * 64 / dt / 1e9 / HBM_PEAK_GBS, 4)
        # the target's measure: weight bytes only (the K/V read is outside it)
        out["decode_8192_weight_read_frac"] = round(weight_bytes * 64 / dt / 1e9 / HBM_PEAK_GBS, 4)
        log(f"decode @8192: {dt / 64 * 1e3:.3f} ms/token, {long_bytes * 64 / dt / 1e9:.0f} GB/s algorithmic")
        r3.close()

    if args.bf16:
        # The reference's deployed precision: the same model with every tensor
        # rounded to BF16 and every matrix (the tied LM head included) uploaded
        # as packed BF16, decode at ctx 454 (the one-launch step when the
        # bridge accepts the all-BF16 plan).
        wb = M.bf16_weights(w)
        mb = E.Model(wb, fmt=E.BF16_EXACT)
        mb.set_run_budget(64 << 30)
        rb = mb.new_run(args.prompt + 80, chunk=args.prompt)
        tok = int(np.argmax(rb.prefill(prompt)))
        for _ in range(2):
            tok = rb.step_greedy(tok)
        mb.sync()
        t = time.perf_counter()
        rb.decode_greedy(tok, 65)
        dt = time.perf_counter() - t
        bf16_bytes = weight_bytes // 2
        out["bf16_decode_454_tok_s"] = round(64 / dt, 2)
        out["bf16_decode_one_launch"] = bool(rb.decode_plan)
        out["bf16_weight_bytes_per_token"] = bf16_bytes
        out["bf16_hbm_weight_read_frac"] = round(bf16_bytes * 64 / dt / 1e9 / HBM_PEAK_GBS, 4)
        log(f"BF16 decode @454: {dt / 64 * 1e3:.3f} ms/token, {bf16_bytes * 64 / dt / 1e9:.0f} GB/s of BF16 weights "
            f"(one-launch: {rb.decode_plan})")
        rb.close()
        # BF16 prefill of the config-3 prompt (one chunk; the engine prepares the
        # BF16 matrices' planes when the bridge offers qr_gemm_bf16_prepare)
        n = 2644
        ids2 = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, n)]
        times = []
        for rep in range(4):
            r2 = mb.new_run(n + 1, chunk=n)
            mb.sync()
            t = time.perf_counter()
            r2.prefill(ids2)
            if rep:
                times.append(time.perf_counter() - t)
            r2.close()
        dt = float(np.median(times))
        out["bf16_prefill_2644_ms"] = round(dt * 1e3, 2)
        out["bf16_prefill_2644_tok_s"] = round(n / dt, 1)
        log(f"BF16 prefill 2644: {dt * 1e3:.1f} ms (median of {len(times)})")
        mb.close()
        del wb

    if args.int8:
        # Config 5: int8 per-row weights (quantised on the host by the engine, as the
        # reference's upload_int8), decode at ctx 454 (the one-launch step when the
        # bridge accepts the int8 plan, else the op sequence) and a 4-row verify
        # with per-row DeltaNet snapshots (verify_rollback_greedy + accept).
        specs = [sp for sp in M.tensor_specs(c) if sp.kind == "matrix"]
        int8_bytes = sum(sp.shape[0] * sp.shape[1] + 4 * sp.shape[0] for sp in specs)
        m8 = E.Model(w, fmt=E.INT8)
        m8.set_run_budget(64 << 30)
        r8 = m8.new_run(args.prompt + 160, chunk=args.prompt, snapshots=3)
        tok = int(np.argmax(r8.prefill(prompt)))
        for _ in range(2):
            tok = r8.step_greedy(tok)
        m8.sync()
        t = time.perf_counter()
        ids8, _ = r8.decode_greedy(tok, 65)
        dt = time.perf_counter() - t
        out["int8_decode_454_tok_s"] = round(64 / dt, 2)
        out["int8_decode_one_launch"] = bool(r8.decode_plan)
        out["int8_weight_bytes_per_token"] = int8_bytes
        out["int8_hbm_weight_read_frac"] = round(int8_bytes * 64 / dt / 1e9 / HBM_PEAK_GBS, 4)
        log(f"int8 decode @454: {dt / 64 * 1e3:.3f} ms/token, {int8_bytes * 64 / dt / 1e9:.0f} GB/s of int8 weights")
        r8.close()
        # int8 prefill of the config-3 prompt (one chunk; the engine prepares the
        # int8 matrices' planes when the bridge offers qr_gemm_i8_prepare)
        n = 2644
        ids2 = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, n)]
        times = []
        for rep in range(4):
            r2 = m8.new_run(n + 1, chunk=n)
            m8.sync()
            t = time.perf_counter()
            r2.prefill(ids2)
            if rep:
                times.append(time.perf_counter() - t)
            r2.close()
        dt = float(np.median(times))
        out["int8_prefill_2644_ms"] = round(dt * 1e3, 2)
        log(f"int8 prefill 2644: {dt * 1e3:.1f} ms (median of {len(times)})")
        out["int8_verify4_ms"] = round(verify4_ms(m8, prompt), 3)
        log(f"int8 4-row verify with snapshots + accept(1): {out['int8_verify4_ms']:.3f} ms")
        if args.spec:
            spec = speculative_rates(E, m8, prompt, 3, 64, 3)
            out["int8_speculative_454"] = spec
            log(f"int8 speculative depth 3: greedy {spec['greedy_tok_s']} tok/s, n-gram {spec['ngram']['tok_s']} "
                f"tok/s, known draft {spec['known']['tok_s']} tok/s")
        m8.close()

    if args.dropin:
        # What an unmodified reference engine would get from this bridge: its
        # fp32 call sequence (one qr_gemv per matrix plus separate norm ops, no
        # one-launch step, a per-token embedding copy) and 128-token prefill
        # chunks (src/device.rs PREFILL_CHUNK).
        md = E.Model(w, disable=E.NO_DECODE_STEP | E.NO_F32_FUSIONS | E.NO_EMBED_ROWS | E.NO_PREPARED_GEMM)
        rd = md.new_run(args.prompt + 64, chunk=PREFILL_CHUNK)
        tok = int(np.argmax(rd.prefill(prompt)))
        for _ in range(3):
            tok = rd.step_greedy(tok)
        md.sync()
        t = time.perf_counter()
        for _ in range(32):
            tok = rd.step_greedy(tok)
        md.sync()
        dt = (time.perf_counter() - t) / 32
        out["decode_454_dropin_tok_s"] = round(1.0 / dt, 2)
        log(f"drop-in decode @454 (op sequence): {dt * 1e3:.3f} ms/token")
        rd.close()
        n = 2644
        ids2 = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, n)]
        times = []
        for rep in range(3):
            r2 = md.new_run(n, chunk=PREFILL_CHUNK)
            md.sync()
            t = time.perf_counter()
            r2.prefill(ids2)
            if rep:
                times.append(time.perf_counter() - t)
            r2.close()
        dt = float(np.median(times))
        out["prefill_2644_chunk128_tok_s"] = round(n / dt, 1)
        log(f"drop-in prefill 2644 in 128-token chunks: {dt * 1e3:.1f} ms")
        md.close()

    # prefill last: measured right after the 10,240-token prefill, the ctx-8192
    # decode took 0.761 ms per token, measured before the prefills 0.743 ms
    if args.prefill:
        # Config 3: one chunk of n uniform random IDs (seed 2) into a fresh run,
        # timed from the call to the last-row logits on the host (as the
        # reference times prefill, src/device/cli.rs:775-791); one untimed run,
        # then the median of `reps`.
        for n, reps in ((2644, 5), (10240, 3)):
            ids2 = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, n)]
            times = []
            for rep in range(reps + 1):
                r2 = model.new_run(n + 1, chunk=n)
                model.sync()
                t = time.perf_counter()
                r2.prefill(ids2)
                dt = time.perf_counter() - t
                if rep:
                    times.append(dt)
                r2.close()
            dt = float(np.median(times))
            proj, attn, rule = prefill_flop_parts(c, n, weight_bytes // 4)
            tflops = (proj + attn + rule) / dt / 1e12
            # the instructions executed: BF16 part products for the
            # projections and attention, fp32 MFMA for the DeltaRule; the
            # fraction of the prefill's time the whole job would take at
            # those peaks
            executed = BF16_PARTS * (proj + attn) / dt / 1e12
            at_peak = BF16_PARTS * (proj + attn) / (MFMA_BF16_PEAK_TFLOPS * 1e12) + rule / (MFMA_F32_PEAK_TFLOPS * 1e12)
            out[f"prefill_{n}_tok_s"] = round(n / dt, 1)
            out[f"prefill_{n}_ms"] = round(dt * 1e3, 2)
            out[f"prefill_{n}_tflops"] = round(tflops, 2)
            out[f"prefill_{n}_bf16_executed_tflops"] = round(executed, 1)
            out[f"prefill_{n}_executed_peak_frac"] = round(at_peak / dt, 4)
            # the fp32-equivalent rate over the fp32 MFMA peak: above 1 once the
            # split-BF16 products outrun fp32 MFMA (not a fraction of any peak
            # the prefill executes against; executed_peak_frac is that)
            out[f"prefill_{n}_fp32_equiv_over_fp32_mfma_peak"] = round(tflops / MFMA_F32_PEAK_TFLOPS, 4)
            log(f"prefill {n}: {dt * 1e3:.1f} ms (median of {reps}), {n / dt:.0f} tok/s, "
                f"{tflops:.1f} TFLOP/s algorithmic fp32; executed {executed:.0f} TFLOP/s of BF16 part products; "
                f"{at_peak / dt:.1%} of the executed instructions' peak time")
    if args.copy_calibration > 0:
        from qwen_mi355x.bridge import Bridge
        br = Bridge()
        n = args.copy_calibration << 18  # floats
        src, dst = br.alloc(n), br.alloc(n)
        br.copy(dst, src, n)
        br.sync()
        out["copy_calibration_bytes"] = n * 4
        del src, dst
        br.close()

    if args.cpu_steps > 0:
        # The oracle (C++ restatement of the reference's Backend::Vector CPU
        # path, one step_compact per token with its logits) on this host, as
        # the reference's benchmark times it (src/benchmark.rs:93-154: one
        # warmup, then measured runs; tok/s = steps / summed step time):
        #   decode: steps at ctx 454 on the config-2 greedy tokens, from the
        #     GPU run's state after the prompt;
        #   prefill: token-by-token steps of the 2644-token prompt (seed 2)
        #     from position 2640, from the GPU's state after its first 2640
        #     tokens (the reference's CPU prefill is one such step per token).
        # Each run starts from a fresh copy of the loaded state.
        import oracle as O
        cpu = host_cpu()
        share = min(cpu["affinity"], 16)
        n2 = 2644
        ids2 = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, n2)]
        start2 = n2 - args.cpu_steps
        loads = {}
        for name, pre in (("decode", prompt), ("prefill", ids2[:start2])):
            rc = model.new_run(len(pre) + 8, chunk=len(pre))
            rc.prefill(pre)
            loads[name] = (len(pre), {(layer, which): rc.state(layer, which)
                                      for layer in range(c.num_layers) for which in range(4)})
            rc.close()
        oracle = O.Oracle(w)
        samples = {"decode": ids[1:1 + args.cpu_steps], "prefill": ids2[start2:start2 + args.cpu_steps]}
        warm_tok = {"decode": ids[0], "prefill": ids2[start2 - 1]}
        rates = {}
        for threads in sorted({min(share, 8), share}):
            O.set_threads(threads)
            for name in ("decode", "prefill"):
                pos, parts = loads[name]
                base = oracle.new_state()
                base.load(pos, lambda layer, which: parts[(layer, which)])
                w0 = base.clone()
                w0.step(warm_tok[name], O.VECTOR)  # warmup (pages the weights in)
                del w0
                runs = []
                for _ in range(args.cpu_runs):
                    st = base.clone()
                    t = time.perf_counter()
                    for tok in samples[name]:
                        st.step(tok, O.VECTOR)
                    runs.append(time.perf_counter() - t)
                    del st
                rates[(name, threads)] = (len(samples[name]) * len(runs) / sum(runs),
                                          [round(len(samples[name]) / r, 3) for r in runs])
                log(f"cpu baseline {name}: {1e3 * sum(runs) / (len(runs) * len(samples[name])):.1f} ms/token on "
                    f"{threads} threads (runs: {rates[(name, threads)][1]} tok/s)")
                del base
        default = min(share, 8)
        out["cpu_baseline"] = {"value": round(rates[("decode", default)][0], 3), "unit": "tok/s", "cores": default,
                               "kind": "port",
                               "sample": f"{args.cpu_runs} runs x {args.cpu_steps} decode steps at ctx {args.prompt + 2}"
                                         f"..{args.prompt + 1 + args.cpu_steps} after one warmup step (config-2 greedy "
                                         "tokens, from the GPU run's state after the prompt), through the CPU oracle's "
                                         "Backend::Vector path (C++ restatement of the reference's Rust CPU decode); "
                                         f"{default} threads = the reference default min(cores, 8); tok/s = steps / "
                                         "summed step time",
                               "runs": rates[("decode", default)][1],
                               "all_cores": {"value": round(rates[("decode", share)][0], 3), "cores": share,
                                             "runs": rates[("decode", share)][1]},
                               "prefill_2644": {"value": round(rates[("prefill", default)][0], 3), "unit": "tok/s",
                                                "cores": default, "runs": rates[("prefill", default)][1],
                                                "all_cores": round(rates[("prefill", share)][0], 3),
                                                "sample": f"{args.cpu_runs} runs x token-by-token steps at positions "
                                                          f"{start2}..{n2 - 1} of the 2644-token prompt (seed 2) "
                                                          "after one warmup step, from the GPU's state after the "
                                                          f"first {start2} tokens (the reference's CPU prefill: one "
                                                          "step with logits per token)"},
                               "host": cpu}

    run.close()
    model.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
