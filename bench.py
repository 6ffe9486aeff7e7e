"""Decode throughput of the LFM2.5-230M-shape BF16 batch-1 hot path on one GPU.

    python bench.py [--steps K] [--warmup W] [--exec persistent|staged] [--prompt P]
    python bench.py --batch B [--steps K]                  (batched decode, B sequences)
    python bench.py --workload encoder --batch B [--steps K] (Parakeet encoder)
    python bench.py --workload w8gemv [--group 0|32|64]    (INT8-weight GEMV)
    python bench.py --weights w8g32 [--steps K]           (decode with 8-bit weights)

Workload (the full decode step, random-init N(0, 0.02) BF16 weights, seed 0):
a 32-token prompt of uniform ids in [0, 65536) is prefilled (untimed), then
K greedy decode tokens run back to back, each consuming the token the
previous one selected on the device. One "step" is one decode token.
W warmup tokens run first on a separate prompt pass. The timed region is
bracketed by device synchronisations and measured with HIP events on the
stream the decode kernel runs on; inputs are resident in HBM.

roofline: algorithmic bytes of the decode call = K * 459,386,368 weight
bytes + the KV bytes read (12,288 B per cached position per token) +
2 KB embedding row per token, divided by the call's time (its two persistent
launches), against MI355X's 8 TB/s HBM peak. traffic: HBM bytes of the call
(K x the measured bytes per token in the committed rocprofv3 counter summary
profiles/decode_traffic.txt), or null without that summary.

The measured process is torch-free (ryzenai-npu-lab_amd/hip.py binds the HIP
runtime with ctypes), so rocprofv3 can trace the cooperative decode launches.
cpu_baseline: a PyTorch-CPU BF16 restatement of the same step
(oracle/torch_cpu.py) decoding the same model token by token on the host
cores, in a child process, at 8 threads and at the physical cores of one
NUMA node (~10 s of decode in total).
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

WEIGHT_BYTES = 459_386_368
KV_BYTES_PER_POSITION = 12_288
EMBED_ROW_BYTES = 2_048
PEAK_GBPS = 8000.0
PROMPT = 32
CAPACITY = 4096  # KV positions per attention head (the largest X8Model tier)
METRIC = "decode tok/s + achieved HBM GB/s (% of peak), LFM2.5-230M-shape bf16 batch 1"
# 8-bit weights: int8 projections and table (q bytes) + one FP32 scale per 32
# weights + the BF16 norms, conv taps and QK norms (110,080 B) per token;
# the embedding row is 1,024 int8 + 32 scales.
W8_WEIGHT_BYTES = 162_529_280 + 20_316_160 + 67_108_864 + 8_388_608 + 110_080
W8_EMBED_ROW_BYTES = 1_024 + 128
W8_METRIC = "decode tok/s + achieved HBM GB/s (% of peak), LFM2.5-230M-shape w8g32 weights batch 1"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--exec", dest="exec_mode", default="persistent",
                    choices=("persistent", "staged"))
    ap.add_argument("--prompt", type=int, default=PROMPT,
                    help="prompt length of the decode workload (the timed tokens attend to it; "
                         "the CPU baseline is skipped beyond 256)")
    ap.add_argument("--batch", type=int, default=1,
                    help="B > 1: B independent sequences decoded in lockstep on the matrix cores "
                         "(lfm25_batch_decode) instead of the batch-1 headline")
    ap.add_argument("--group", type=int, default=32, choices=(0, 32, 64),
                    help="w8gemv: inputs per FP32 scale (0: one scale per row)")
    ap.add_argument("--workload", choices=("decode", "encoder", "w8gemv", "gemv", "conv-layer", "attn-layer",
                                           "prefill"),
                    default="decode",
                    help="decode: the LFM2.5 decode hot path (default); encoder: the Parakeet "
                         "encoder over --batch 10 s windows; gemv / conv-layer / attn-layer: one "
                         "kernel call per step (configs 1 / 2 / 3) over >= 512 MB of weight copies")
    ap.add_argument("--weights", default="bf16", choices=("bf16", "w8g32"),
                    help="decode: weight format (w8g32: every projection and the tied table as int8 "
                         "with one FP32 scale per row and 32 inputs, lfm25_decode_w8)")
    ap.add_argument("--context", type=int, default=1024,
                    help="attn-layer: positions attended (the token sits at context - 1), 1..4096")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def traffic_from_profile():
    path = ROOT / "profiles" / "decode_traffic.txt"
    if not path.exists():
        return None
    m = re.search(r"^hbm_bytes_per_token:\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(prompt, seconds):
    """The PyTorch-CPU BF16 restatement of the decode step (oracle/torch_cpu.py,
    the reference's CPU path: experiments/010_cpu_greedy.py:39-63) on the
    same synthetic model and prompt, in a child process so this process stays
    torch-free: token-by-token greedy decode with conv / KV caches, median
    step time over >= 32 steps after 3 warm-up steps, at 8 threads (the
    reference's setting) and at the physical cores of one NUMA node this
    process may use. `value` is the NUMA-node figure."""
    import subprocess
    from oracle.torch_cpu import physical_cores_of_one_numa_node
    node = physical_cores_of_one_numa_node()
    threads = [8] if node == 8 else [8, node]
    cmd = [sys.executable, "-m", "oracle.torch_cpu", "--threads", *map(str, threads),
           "--seconds", f"{max(seconds / len(threads), 1.0):.2f}", "--prompt", str(len(prompt))]
    proc = subprocess.run(cmd, cwd=str(ROOT), capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        raise RuntimeError(f"CPU baseline failed: {proc.stderr[-2000:]}")
    runs = [json.loads(line) for line in proc.stdout.splitlines() if line.startswith("{")]
    main = next(r for r in runs if r["threads"] == threads[-1])
    return {"value": main["tok_s"], "unit": "tok/s", "cores": main["threads"], "kind": "port",
            "sample": f"{main['steps']} greedy decode steps after a {len(prompt)}-token prompt, PyTorch "
                      f"{main['torch']} BF16 on the CPU (median step {main['ms_median']} ms); physical cores "
                      f"of one NUMA node: {node}",
            "runs": [{"cores": r["threads"], "value": r["tok_s"], "ms_median": r["ms_median"],
                      "ms_p10": r["ms_p10"], "ms_p90": r["ms_p90"], "steps": r["steps"]} for r in runs]}


def run_decode(args, lab, prompt):
    """Upload the model, prefill the prompt, time `args.steps` decode tokens.
    Returns (ms, wall_s, status, checkpoint). Torch-free: device buffers and
    events come from the HIP runtime directly, so the measured process holds
    nothing but the runtime and the decode library."""
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    W = lab.weights
    lib = lab._lib.load(bind_torch=False)
    if hip.device_count() < 1:
        raise SystemExit("no GPU visible")
    t0 = time.perf_counter()
    ck = W.synthetic_checkpoint(0)
    stream = W.pack_stream(ck)
    if stream.size != lib.lfm25_weights_elems():
        raise RuntimeError("packed weight stream does not match the library layout")
    table = ck["model.embed_tokens.weight"]
    cap = CAPACITY
    conv_layers, attn_layers = W.KINDS.count("conv"), W.KINDS.count("attention")
    bufs = {
        "weights": hip.Buffer.from_array(stream),
        "embedding": hip.Buffer.from_array(table),
        "rope": hip.Buffer.from_array(W.rope_table(cap)),
        "conv": hip.Buffer.zeros(conv_layers * W.HIDDEN * 3 * 2),
        "keys": hip.Buffer.zeros(attn_layers * W.KV_HEADS * cap * W.HEAD_DIM * 2),
        "values": hip.Buffer.zeros(attn_layers * W.KV_HEADS * cap * W.HEAD_DIM * 2),
        "workspace": hip.Buffer.zeros(lib.lfm25_decoder_workspace_bytes()),
        "tokens_in": hip.Buffer.from_array(np.asarray(prompt, np.int32)),
        "tokens_out": hip.Buffer(4 * max(args.steps, args.warmup, 1)),
    }
    desc = lab._lib.Decoder(bufs["weights"].ptr, bufs["embedding"].ptr, bufs["rope"].ptr,
                            bufs["conv"].ptr, bufs["keys"].ptr, bufs["values"].ptr,
                            bufs["workspace"].ptr, cap, int(table.shape[0]))
    exec_mode = lab._lib.EXEC_PERSISTENT if args.exec_mode == "persistent" else lab._lib.EXEC_STAGED
    if exec_mode == lab._lib.EXEC_PERSISTENT:
        lab._lib.call("lfm25_init")  # the one-time placement probe, outside every timed region
    w8 = None
    if args.weights == "w8g32":
        layers, tq, ts = W.pack_w8(ck)
        if layers.size != lib.lfm25_w8_layers_bytes():
            raise RuntimeError("8-bit weight stream does not match the library layout")
        bufs["w8_layers"] = hip.Buffer.from_array(layers)
        bufs["w8_table"] = hip.Buffer.from_array(tq)
        bufs["w8_scales"] = hip.Buffer.from_array(ts)
        w8 = lab._lib.W8Model(bufs["w8_layers"].ptr, bufs["w8_table"].ptr, bufs["w8_scales"].ptr)

    def reset():
        lab._lib.call("lfm25_decoder_reset", desc, None)

    def decode(n_in, n_gen, tokens_in):
        if w8 is not None:
            lab._lib.call("lfm25_decode_w8", desc, w8, tokens_in, n_in, n_gen, bufs["tokens_out"].ptr, None)
        else:
            lab._lib.call("lfm25_decode", desc, tokens_in, n_in, n_gen, bufs["tokens_out"].ptr,
                          exec_mode, None)

    hip.synchronize()
    print(f"# model ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    if args.warmup > 0:
        reset()
        decode(len(prompt), args.warmup, bufs["tokens_in"].ptr)
    reset()
    decode(len(prompt), 1, bufs["tokens_in"].ptr)  # selects the first reply token
    hip.synchronize()
    start, end = hip.Event(), hip.Event()
    wall0 = time.perf_counter()
    start.record()
    decode(1, args.steps, None)                    # consumes the token held on the device
    end.record()
    end.synchronize()
    wall = time.perf_counter() - wall0
    status = int(bufs["workspace"].download(np.int32, 3)[2])
    ms = start.elapsed_ms(end)
    del bufs
    return ms, wall, status, ck


BATCH_METRIC = "batched decode tok/s (B independent sequences, lockstep), LFM2.5-230M-shape bf16"


def run_batched(args, lab):
    """B sequences, each with its own 32-token prompt (prefilled in passes of
    up to 64 rows, untimed), then `args.steps` lockstep decode steps timed as
    one lfm25_batch_decode call. Torch-free like run_decode."""
    import ctypes
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    W = lab.weights
    lib = lab._lib.load(bind_torch=False)
    B = args.batch
    ck = W.synthetic_checkpoint(0)
    stream = W.pack_stream(ck)
    table = ck["model.embed_tokens.weight"]
    cap = PROMPT + args.steps + args.warmup + 1
    conv_layers, attn_layers = W.KINDS.count("conv"), W.KINDS.count("attention")
    kv = B * attn_layers * W.KV_HEADS * cap * W.HEAD_DIM * 2
    bufs = {
        "weights": hip.Buffer.from_array(stream),
        "embedding": hip.Buffer.from_array(table),
        "rope": hip.Buffer.from_array(W.rope_table(cap)),
        "conv": hip.Buffer.zeros(B * conv_layers * W.HIDDEN * 3 * 2),
        "keys": hip.Buffer.zeros(kv),
        "values": hip.Buffer.zeros(kv),
        "workspace": hip.Buffer.zeros(lib.lfm25_batch_workspace_bytes()),
        "tokens": hip.Buffer(4 * 64),
        "out": hip.Buffer(4 * B * max(args.steps, args.warmup, 1)),
    }
    desc = lab._lib.Batch(bufs["weights"].ptr, bufs["embedding"].ptr, bufs["rope"].ptr, bufs["conv"].ptr,
                          bufs["keys"].ptr, bufs["values"].ptr, bufs["workspace"].ptr, B, cap,
                          int(table.shape[0]))
    prompts = [[int(t) for t in lab.rng.uniform_ints(0, f"bench.batch.prompt{s}", PROMPT, 16)]
               for s in range(B)]
    queue = [(prompts[s][i], s, i) for s in range(B) for i in range(PROMPT)]
    while queue:
        chunk, queue = queue[:64], queue[64:]
        rows = np.asarray(chunk, np.int32)
        lab._lib.call("lfm25_batch_pass", ctypes.byref(desc), rows.ctypes.data, len(rows), 1,
                      bufs["tokens"].ptr, None, None)
        last = [m for m, (_, s, i) in enumerate(chunk) if i == PROMPT - 1]
        if last:
            got = bufs["tokens"].download(np.int32, len(chunk))
            for m in last:
                prompts[chunk[m][1]].append(int(got[m]))
    first = hip.Buffer.from_array(np.asarray([p[-1] for p in prompts], np.int32))
    pos = np.full(B, PROMPT, np.int32)
    if args.warmup > 0:
        lab._lib.call("lfm25_batch_decode", ctypes.byref(desc), first.ptr, pos.ctypes.data, args.warmup,
                      bufs["out"].ptr, None)
        pos = pos + args.warmup
    hip.synchronize()
    start, end = hip.Event(), hip.Event()
    wall0 = time.perf_counter()
    start.record()
    lab._lib.call("lfm25_batch_decode", ctypes.byref(desc), first.ptr, pos.ctypes.data, args.steps,
                  bufs["out"].ptr, None)
    end.record()
    end.synchronize()
    wall = time.perf_counter() - wall0
    status = int(bufs["workspace"].download(np.int32, 1)[0])
    ms = start.elapsed_ms(end)
    ctx0 = int(pos[0]) + 1
    del bufs
    return ms, wall, status, ctx0


def main_batched(args, lab):
    B, steps = args.batch, args.steps
    ms, wall, status, ctx0 = run_batched(args, lab)
    if status:
        print(f"batched decode status 0x{status:x}", file=sys.stderr)
        return 1
    kv = B * sum(KV_BYTES_PER_POSITION * (ctx0 + i) for i in range(steps))
    algo = steps * (WEIGHT_BYTES + B * EMBED_ROW_BYTES) + kv
    achieved = algo / (ms * 1e-3) / 1e9
    line = {
        "metric": BATCH_METRIC,
        "value": round(B * steps / (ms * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, uniform prompt ids, seed 0)",
        "config": {"workload": f"LFM2.5-230M-shape greedy decode of {B} independent sequences in lockstep, "
                               f"{PROMPT}-token prompts then {steps} steps "
                               + ("(persistent batched decode)" if B in (2, 4, 8)
                                  else "(persistent batched decode below 256 positions, batched MFMA pass after)"
                                  if B == 16 else "(batched MFMA pass)"),
                   "batch": B, "prompt": PROMPT, "decode_steps": steps},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4), "traffic": None},
        "wall_ms": round(wall * 1e3, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


ENCODER_METRIC = "Parakeet-0.6B-shape encoder windows/s (24 FastConformer blocks, 125 frames = 10 s), bf16"
ENCODER_LAYERS = 24
ENCODER_FRAMES = 128  # one padded block
ENCODER_VALID = 125
# GEMM FLOPs of one 125-frame window: 24 blocks x 125 frames x 2 x the block's
# multiply-adds per frame (FFN 2 x 2 x 1024 x 4096, q|k|v 3 x 1024^2, out
# 1024^2, pw1 2 x 1024^2, pw2 1024^2)
ENCODER_FLOP = 2 * ENCODER_VALID * ENCODER_LAYERS * (4 * 1024 * 4096 + 7 * 1024 * 1024)
MFMA_BF16_PEAK_TFLOPS = 2500.0


def run_encoder(args, lab):
    """`args.batch` windows of 125 N(0,1) frames (padded to 128) through 24
    random-init blocks, `args.steps` times back to back on the device (each
    pass runs on the previous pass's output, in place); torch-free."""
    import ctypes
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    pk = importlib.import_module("ryzenai-npu-lab_amd.parakeet")
    lib = lab._lib.load(bind_torch=False)
    B = args.batch
    bufs, descs, weight_bytes, cpu_layers = [], [], 0, []
    for i in range(ENCODER_LAYERS):
        w, pos = pk.synthetic_layer(0, i)
        if i < 2:
            cpu_layers.append((w, pos))
        packed = {k: hip.Buffer.from_array(v) for k, v in pk.pack_layer(w, pos).items()}
        weight_bytes += sum(v.nbytes for k, v in packed.items() if k != "pos")
        bufs.append(packed)
        descs.append(lab._lib.PkLayer(*[packed[f].ptr for f, _ in lab._lib.PkLayer._fields_]))
    layers = (lab._lib.PkLayer * ENCODER_LAYERS)(*descs)
    rng = np.random.default_rng(0)
    x0 = np.zeros((B, ENCODER_FRAMES, 1024), np.float32)
    x0[:, :ENCODER_VALID] = rng.standard_normal((B, ENCODER_VALID, 1024), dtype=np.float32)
    x = hip.Buffer.from_array(pk._bits(x0))
    ws = hip.Buffer.zeros(lib.lfm25_pk_workspace_bytes(B, ENCODER_FRAMES))

    def run(n):
        for _ in range(n):
            lab._lib.call("lfm25_pk_encoder", layers, ENCODER_LAYERS, x.ptr, B, ENCODER_FRAMES, ENCODER_VALID,
                          ws.ptr, None)

    run(args.warmup)
    hip.synchronize()
    start, end = hip.Event(), hip.Event()
    wall0 = time.perf_counter()
    start.record()
    run(args.steps)
    end.record()
    end.synchronize()
    wall = time.perf_counter() - wall0
    out = x.download(np.uint16, B * ENCODER_FRAMES * 1024)
    finite = bool(np.isfinite(pk.bf16_bits_to_f32(out)).all())
    ms = start.elapsed_ms(end)
    del bufs, x, ws
    return ms, wall, finite, weight_bytes, cpu_layers, x0[0]


def encoder_cpu_baseline(layers, x, seconds):
    """The oracle's BF16 mirror of one block (numpy), cycled over the sample
    layers on one 128-frame window for ~`seconds`; scaled to 24 blocks."""
    from oracle import parakeet as P
    try:
        from threadpoolctl import threadpool_info
        threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
    except ImportError:
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    xb, n, t0 = P.r(x), 0, time.perf_counter()
    while True:
        w, pos = layers[n % len(layers)]
        xb, _ = P.block_bf16(xb, w, pos, ENCODER_VALID)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or n >= 240:
            break
    per_window = el / n * ENCODER_LAYERS
    return {"value": round(1.0 / per_window, 4), "unit": "windows/s", "cores": threads, "kind": "port",
            "sample": f"{n} Conformer blocks of one 125-frame window (numpy BF16 mirror, {el:.1f} s), "
                      f"x {ENCODER_LAYERS} blocks per window"}


def main_encoder(args, lab):
    B, steps = args.batch, args.steps
    ms, wall, finite, weight_bytes, cpu_layers, x0 = run_encoder(args, lab)
    if not finite:
        print("encoder output is not finite", file=sys.stderr)
        return 1
    step_s = ms * 1e-3 / steps
    if B == 1:
        achieved = weight_bytes / step_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBPS, 4), "traffic": None}
    else:
        achieved = B * ENCODER_FLOP / step_s / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None}
    line = {
        "metric": ENCODER_METRIC,
        "value": round(B / step_s, 2),
        "unit": "windows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, N(0,1) frames, seed 0)",
        "config": {"workload": f"Parakeet-0.6B-shape encoder, {ENCODER_LAYERS} blocks, batch {B} windows of "
                               f"{ENCODER_VALID} frames padded to {ENCODER_FRAMES}",
                   "batch": B, "frames": ENCODER_VALID, "blocks": ENCODER_LAYERS,
                   "weight_bytes": weight_bytes, "gemm_flop_per_window": ENCODER_FLOP},
        "roofline": roof,
        "wall_ms": round(wall * 1e3, 3),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = encoder_cpu_baseline(cpu_layers, x0, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


PREFILL_ROWS = 64  # prompt positions per matrix-core pass


def main_prefill(args, lab):
    """Time to first token of a `--prompt P` prompt, as X8Model.prefill runs it:
    the P - 1 tokens before the last in matrix-core passes of up to 64 rows
    (lfm25_batch_pass on the decoder's caches), then one decode step that
    consumes the last token and selects the first reply token. Also timed:
    the same prompt token by token through the persistent decode. Each
    variant runs once untimed, then `--steps` times from a reset state."""
    import ctypes
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    W = lab.weights
    lib = lab._lib.load(bind_torch=False)
    P = args.prompt
    ck = W.synthetic_checkpoint(0)
    stream = W.pack_stream(ck)
    table = ck["model.embed_tokens.weight"]
    cap = CAPACITY
    conv_layers, attn_layers = W.KINDS.count("conv"), W.KINDS.count("attention")
    prompt = [int(t) for t in lab.rng.uniform_ints(0, "bench.prefill.prompt", P, 16)]
    bufs = {
        "weights": hip.Buffer.from_array(stream), "embedding": hip.Buffer.from_array(table),
        "rope": hip.Buffer.from_array(W.rope_table(cap)),
        "conv": hip.Buffer.zeros(conv_layers * W.HIDDEN * 3 * 2),
        "keys": hip.Buffer.zeros(attn_layers * W.KV_HEADS * cap * W.HEAD_DIM * 2),
        "values": hip.Buffer.zeros(attn_layers * W.KV_HEADS * cap * W.HEAD_DIM * 2),
        "workspace": hip.Buffer.zeros(lib.lfm25_decoder_workspace_bytes()),
        "batch_ws": hip.Buffer.zeros(lib.lfm25_batch_workspace_bytes()),
        "tokens_in": hip.Buffer.from_array(np.asarray(prompt, np.int32)),
        "last": hip.Buffer.from_array(np.asarray(prompt[-1:], np.int32)),
        "tokens_out": hip.Buffer(64),
    }
    b = {k: v.ptr for k, v in bufs.items()}
    desc = lab._lib.Decoder(b["weights"], b["embedding"], b["rope"], b["conv"], b["keys"], b["values"],
                            b["workspace"], cap, int(table.shape[0]))
    batch = lab._lib.Batch(b["weights"], b["embedding"], b["rope"], b["conv"], b["keys"], b["values"],
                           b["batch_ws"], 1, cap, int(table.shape[0]))
    ctl = np.zeros(1, np.int32)
    tables = []
    for start in range(0, P - 1, PREFILL_ROWS):
        chunk = prompt[start:min(start + PREFILL_ROWS, P - 1)]
        tables.append(np.asarray([(t, 0, start + i) for i, t in enumerate(chunk)], np.int32))

    def batched():
        lab._lib.call("lfm25_decoder_reset", desc, None)
        for rows in tables:
            lab._lib.call("lfm25_batch_pass", ctypes.byref(batch), rows.ctypes.data, len(rows), 0, None, None, None)
        ctl[0] = P - 1
        bufs["workspace"].upload(ctl)  # the position the decode continues from (host-ordered: a blocking copy)
        lab._lib.call("lfm25_decode", desc, b["last"], 1, 1, b["tokens_out"], lab._lib.EXEC_PERSISTENT, None)

    def token_by_token():
        lab._lib.call("lfm25_decoder_reset", desc, None)
        lab._lib.call("lfm25_decode", desc, b["tokens_in"], P, 1, b["tokens_out"], lab._lib.EXEC_PERSISTENT, None)

    results = {}
    for name, fn in (("batched", batched), ("token_by_token", token_by_token)):
        fn()
        hip.synchronize()
        times = []
        for _ in range(args.steps):
            start, end = hip.Event(), hip.Event()
            hip.synchronize()
            t0 = time.perf_counter()
            start.record()
            fn()
            end.record()
            end.synchronize()
            times.append((start.elapsed_ms(end), (time.perf_counter() - t0) * 1e3))
        status = int(bufs["workspace"].download(np.int32, 3)[2]) | int(bufs["batch_ws"].download(np.int32, 1)[0])
        if status:
            print(f"prefill ({name}) status 0x{status:x}", file=sys.stderr)
            return 1
        tok = int(bufs["tokens_out"].download(np.int32, 1)[0])
        ev = sorted(t[0] for t in times)
        wall = sorted(t[1] for t in times)
        results[name] = {"ms": ev[len(ev) // 2], "wall_ms": wall[len(wall) // 2], "first_token": tok}
    ms = results["batched"]["ms"]
    line = {
        "metric": f"time to first token (ms), {P}-token prompt, LFM2.5-230M-shape bf16 batch 1",
        "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": 1,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (random-init N(0,0.02) weights, uniform prompt ids, seed 0)",
        "config": {"workload": f"prompt of {P} uniform ids: {P - 1} in matrix-core passes of up to "
                               f"{PREFILL_ROWS} rows, the last in one decode step that selects the first token",
                   "prompt": P, "passes": len(tables)},
        "prompt_tok_s": round(P / (ms * 1e-3), 1),
        "token_by_token_ms": round(results["token_by_token"]["ms"], 3),
        "first_tokens": [results["batched"]["first_token"], results["token_by_token"]["first_token"]],
        "wall_ms": round(results["batched"]["wall_ms"], 3),
    }
    print(json.dumps(line), flush=True)
    del bufs
    return 0


ROTATE_BYTES = 512 << 20  # distinct weight copies cycled per timed loop: past the 256 MB Infinity Cache


def _bits(a):
    """float32 -> BF16 bit patterns (round to nearest even)."""
    import numpy as np
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _timed(hip, launch, copies, steps, warmup):
    """`warmup` then `steps` launches cycling over `copies`, back to back;
    returns the event-timed milliseconds of the timed launches."""
    for i in range(warmup):
        launch(i % copies)
    hip.synchronize()
    start, end = hip.Event(), hip.Event()
    start.record()
    for i in range(steps):
        launch(i % copies)
    end.record()
    end.synchronize()
    return start.elapsed_ms(end)


def _kernel_line(metric, args, ms, unit_bytes, workload, extra_config, parity):
    per = ms / args.steps
    achieved = unit_bytes / (per * 1e-3) / 1e9
    return {
        "metric": metric, "value": round(per * 1e3, 3), "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(per, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights)",
        "config": {"workload": workload, **extra_config},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBPS, 4), "traffic": None},
        "parity": parity,
    }


def main_gemv(args, lab):
    """Config 1: fused RMSNorm + BF16 GEMV, W [3072 x 1024] (lfm25_norm_bf16_gemv,
    the reference's norm_bf16_gemv), one launch per step over distinct copies
    of the packed [gamma | pad | W] totalling >= 512 MB."""
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    lib = lab._lib.load(bind_torch=False)
    M, K = 3072, 1024
    x = lab.rng.normal_bf16(1, "config1.x", K)
    g = lab.rng.normal_bf16(1, "config1.gamma", K, 1.0, 0.02)
    w = lab.rng.normal_bf16(1, "config1.w", M * K, 0.0, 0.02)
    packed = np.concatenate([g, np.zeros(4096 - K, np.uint16), w])
    copies = -(-ROTATE_BYTES // packed.nbytes)
    bufs = [hip.Buffer.from_array(packed) for _ in range(copies)]
    bx, by = hip.Buffer.from_array(x), hip.Buffer(2 * M)
    launch = lambda i: lab._lib.call("lfm25_norm_bf16_gemv", bx.ptr, bufs[i].ptr, by.ptr, M, K, None)  # noqa: E731
    ms = _timed(hip, launch, copies, args.steps, args.warmup)
    y = by.download(np.uint16, M)
    parity = None
    if not args.no_cpu:
        from oracle import lfm25 as O
        want = O.linear(w.reshape(M, K), O.rms_norm(O.f32(x), O.f32(g)))
        got = O.f32(y)
        parity = {"rows_differing": float(np.mean(got != want)),
                  "max_abs_diff": float(np.max(np.abs(got - want)))}
    unit = 6_291_456 + 4_096 + 6_144  # W, x and gamma, y
    line = _kernel_line("fused RMSNorm + BF16 GEMV time per call (us), 3072x1024", args, ms, unit,
                        "config 1: lfm25_norm_bf16_gemv, W 3072x1024, x and gamma of 1024",
                        {"rows": M, "cols": K, "copies": copies, "bytes_per_call": unit}, parity)
    print(json.dumps(line), flush=True)
    return 0


def _layer_copy(lab, kind, seed, capacity):
    """One layer's tensors as separate host arrays (BF16 bits): weights N(0,
    0.02), norms 1 + N(0, 0.02); conv: a state N(0, 1); attention: q|k|v
    contiguous and caches pre-filled N(0, 1)."""
    import numpy as np
    r = lab.rng
    t = {"op_norm": r.normal_bf16(seed, "layer.op_norm", 1024, 1.0, 0.02),
         "ffn_norm": r.normal_bf16(seed, "layer.ffn_norm", 1024, 1.0, 0.02),
         "out": r.normal_bf16(seed, "layer.out", 1024 * 1024, 0.0, 0.02),
         "w1": r.normal_bf16(seed, "layer.w1", 2560 * 1024, 0.0, 0.02),
         "w3": r.normal_bf16(seed, "layer.w3", 2560 * 1024, 0.0, 0.02),
         "w2": r.normal_bf16(seed, "layer.w2", 1024 * 2560, 0.0, 0.02)}
    if kind == "conv":
        t["mixer"] = r.normal_bf16(seed, "layer.in_proj", 3072 * 1024, 0.0, 0.02)
        t["conv_weight"] = r.normal_bf16(seed, "layer.conv", 1024 * 3, 0.0, 0.02)
        t["state"] = r.normal_bf16(seed, "layer.state", 1024 * 3)
    else:
        t["mixer"] = r.normal_bf16(seed, "layer.qkv", 2048 * 1024, 0.0, 0.02)
        t["q_norm"] = r.normal_bf16(seed, "layer.q_norm", 64, 1.0, 0.02)
        t["k_norm"] = r.normal_bf16(seed, "layer.k_norm", 64, 1.0, 0.02)
        kv = 8 * capacity * 64
        t["keys"] = r.normal_bf16(seed, "layer.keys", kv)
        t["values"] = r.normal_bf16(seed, "layer.values", kv)
    return t


def main_layer(args, lab):
    """Config 2 (conv layer) / config 3 (attention layer at --context T): one
    decoder layer per call (lfm25_decode_layer, one cooperative launch),
    cycling over distinct copies of the layer's weights (and, for attention,
    of its pre-filled KV cache) totalling >= 512 MB. Attention: the token at
    position T - 1 appends its row and attends to T positions."""
    import ctypes
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    lib = lab._lib.load(bind_torch=False)
    W = lab.weights
    kind = "conv" if args.workload == "conv-layer" else "attention"
    T = args.context
    capacity = T if kind == "attention" else 1
    host = _layer_copy(lab, kind, 3, capacity)
    weight_keys = [k for k in host if k not in ("state", "keys", "values")]
    weight_bytes = sum(host[k].nbytes for k in weight_keys)
    copies = -(-ROTATE_BYTES // weight_bytes)
    rope = hip.Buffer.from_array(W.rope_table(max(capacity, 1))) if kind == "attention" else None
    layers, keep = [], []
    state_out = hip.Buffer(2 * 1024 * 3)  # the input states stay as uploaded, so every call sees the same one
    for _ in range(copies):
        d = {k: hip.Buffer.from_array(v) for k, v in host.items()}
        keep.append(d)
        L = lab._lib.Layer(kind=lab._lib.LAYER_CONV if kind == "conv" else lab._lib.LAYER_ATTN,
                           op_norm=d["op_norm"].ptr, mixer=d["mixer"].ptr, out=d["out"].ptr,
                           ffn_norm=d["ffn_norm"].ptr, w1=d["w1"].ptr, w3=d["w3"].ptr, w2=d["w2"].ptr)
        if kind == "conv":
            L.conv_weight, L.conv_state_in, L.conv_state_out = d["conv_weight"].ptr, d["state"].ptr, state_out.ptr
        else:
            L.q_norm, L.k_norm = d["q_norm"].ptr, d["k_norm"].ptr
            L.key_cache, L.value_cache, L.rope, L.capacity = d["keys"].ptr, d["values"].ptr, rope.ptr, capacity
        layers.append(L)
    x = lab.rng.normal_bf16(3, "layer.hidden", 1024)
    bx, by = hip.Buffer.from_array(x), hip.Buffer(2048)
    ws = hip.Buffer.zeros(lib.lfm25_decoder_workspace_bytes())
    pos = T - 1 if kind == "attention" else 0

    def launch(i):
        lab._lib.call("lfm25_decode_layer", ctypes.byref(layers[i]), bx.ptr, by.ptr, pos, ws.ptr, None)

    ms = _timed(hip, launch, copies, args.steps, args.warmup)
    status = int(ws.download(np.int32, 3)[2])
    if status:
        print(f"layer status 0x{status:x}", file=sys.stderr)
        return 1
    parity = None
    if not args.no_cpu:
        from oracle import lfm25 as O
        got = O.f32(by.download(np.uint16, 1024))
        want = _layer_oracle(O, host, kind, x, pos, capacity)
        scale = float(np.max(np.abs(want)))
        ulp = 2.0 ** (np.floor(np.log2(scale)) - 7)
        parity = {"max_abs_diff_ulps_of_scale": float(np.max(np.abs(got - want)) / ulp)}
    unit = weight_bytes + 4096 + (12_288 if kind == "conv" else 2048 * (T - 1) + 2048)
    extra = {"kind": kind, "copies": copies, "bytes_per_call": unit, "weight_bytes": weight_bytes}
    if kind == "attention":
        extra["context"] = T
    name = ("config 2: one gated short-conv decode layer (lfm25_decode_layer)" if kind == "conv" else
            f"config 3: one GQA attention decode layer at context {T} (lfm25_decode_layer)")
    metric = ("decode layer time per call (us), LFM2.5-230M-shape " +
              ("conv layer" if kind == "conv" else f"attention layer, context {T}"))
    print(json.dumps(_kernel_line(metric, args, ms, unit, name, extra, parity)), flush=True)
    return 0


def _layer_oracle(O, host, kind, x, pos, capacity):
    """The oracle's layer on the inputs every timed call saw (the conv state
    is written to a separate buffer, so the input state never changes)."""
    import numpy as np
    ck = {}
    names = O.layer_tensor_names(0 if kind == "conv" else 2)
    if kind == "conv":
        vals = [host["op_norm"], host["mixer"].reshape(3072, 1024), host["conv_weight"].reshape(1024, 1, 3),
                host["out"].reshape(1024, 1024), host["ffn_norm"], host["w1"].reshape(2560, 1024),
                host["w3"].reshape(2560, 1024), host["w2"].reshape(1024, 2560)]
    else:
        m = host["mixer"].reshape(2048, 1024)
        vals = [host["op_norm"], m[:1024], m[1024:1536], m[1536:], host["q_norm"], host["k_norm"],
                host["out"].reshape(1024, 1024), host["ffn_norm"], host["w1"].reshape(2560, 1024),
                host["w3"].reshape(2560, 1024), host["w2"].reshape(1024, 2560)]
    ck.update(dict(zip(names, vals)))
    orc = O.Oracle(ck, capacity=max(capacity, 1), layers=3 if kind == "attention" else 1)
    if kind == "conv":
        orc.conv_states[0] = O.f32(host["state"]).reshape(1024, 3)
        return orc.layer(0, O.f32(x), 0, 0)
    orc.keys[0][:, :pos] = O.f32(host["keys"]).reshape(8, capacity, 64)[:, :pos]
    orc.values[0][:, :pos] = O.f32(host["values"]).reshape(8, capacity, 64)[:, :pos]
    orc.position = pos
    return orc.layer(2, O.f32(x), 0, 0)


W8_ROWS, W8_COLS = 65536, 1024  # the tied vocabulary head, the model's largest matrix


def run_w8(args, lab):
    """INT8-weight GEMV over the head's shape (65,536 x 1,024, quantized from
    N(0, 0.02) BF16 weights as the reference's w8 formats do), `args.steps`
    launches back to back on the device; torch-free."""
    import numpy as np
    hip = importlib.import_module("ryzenai-npu-lab_amd.hip")
    lib = lab._lib.load(bind_torch=False)
    rng = np.random.default_rng(0)
    w = (0.02 * rng.standard_normal((W8_ROWS, W8_COLS), dtype=np.float32)).view(np.uint32)
    w_bits = ((w + 0x7FFF + ((w >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even
    q, sc = lab.weights.quantize_w8(w_bits, args.group)
    xv = rng.standard_normal(W8_COLS, dtype=np.float32).view(np.uint32)
    x = ((xv + 0x7FFF + ((xv >> 16) & 1)) >> 16).astype(np.uint16)
    # distinct copies of the quantized matrix, >= 512 MB in all, cycled so
    # that no launch finds its weights in the 256 MB Infinity Cache
    copies = -(-ROTATE_BYTES // (q.nbytes + sc.nbytes))
    bq = [hip.Buffer.from_array(q) for _ in range(copies)]
    bs = [hip.Buffer.from_array(sc) for _ in range(copies)]
    bx, by = hip.Buffer.from_array(x), hip.Buffer(2 * W8_ROWS)

    def launch(i):
        lab._lib.call("lfm25_w8_gemv", bq[i].ptr, bs[i].ptr, bx.ptr, by.ptr, W8_ROWS, W8_COLS, args.group, None)

    ms = _timed(hip, launch, copies, args.steps, args.warmup)
    y = by.download(np.uint16, W8_ROWS)
    nbytes = q.nbytes + sc.nbytes + x.nbytes + 2 * W8_ROWS
    del bq, bs, bx, by
    return ms, nbytes, q, sc, x, y, copies


def main_w8(args, lab):
    import numpy as np
    ms, nbytes, q, sc, x, y, copies = run_w8(args, lab)
    step_s = ms * 1e-3 / args.steps
    achieved = nbytes / step_s / 1e9
    line = {
        "metric": "INT8-weight GEMV GB/s (w8 formats), 65536x1024",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights, bf16 activations, fp32 sums",
        "data": "synthetic (N(0, 0.02) weights quantized, N(0, 1) activation, seed 0)",
        "config": {"workload": f"w8 GEMV {W8_ROWS}x{W8_COLS}, group {args.group or 'row'}, cycling over "
                               f"{copies} weight copies (no launch reads from the Infinity Cache)",
                   "rows": W8_ROWS, "cols": W8_COLS, "group": args.group, "bytes_per_launch": nbytes,
                   "copies": copies},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBPS, 4), "traffic": None},
    }
    if not args.no_cpu:
        oracle = importlib.import_module("oracle.lfm25")
        rows = 4096
        t0 = time.perf_counter()
        n = 0
        while True:
            want = oracle.linear_w8(q[:rows], sc[:rows], args.group, oracle.f32(x))
            n += 1
            if time.perf_counter() - t0 > min(args.cpu_seconds, 5.0):
                break
        cpu_s = (time.perf_counter() - t0) / n
        got = oracle.f32(y[:rows])
        line["cpu_baseline"] = {"value": round(q[:rows].nbytes / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1,
                                "kind": "port", "sample": f"oracle linear_w8 over the first {rows} rows"}
        line["parity_rows_differing"] = float(np.mean(got != want))
    print(json.dumps(line), flush=True)
    return 0


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path "
              "(independent sequences would shard data-parallel, one decoder per GPU)",
              file=sys.stderr)
        return 2
    lab = importlib.import_module("ryzenai-npu-lab_amd")
    if args.workload == "w8gemv":
        return main_w8(args, lab)
    if args.workload == "gemv":
        return main_gemv(args, lab)
    if args.workload == "prefill":
        if not 2 <= args.prompt <= CAPACITY - 1:
            print(f"--prompt must be in [2, {CAPACITY - 1}]", file=sys.stderr)
            return 2
        return main_prefill(args, lab)
    if args.workload in ("conv-layer", "attn-layer"):
        if not 1 <= args.context <= CAPACITY:
            print(f"--context must be in [1, {CAPACITY}]", file=sys.stderr)
            return 2
        return main_layer(args, lab)
    if args.workload == "encoder":
        if not 1 <= args.batch <= 64:
            print("--batch must be in [1, 64]", file=sys.stderr)
            return 2
        return main_encoder(args, lab)
    if args.batch != 1:
        if not 1 <= args.batch <= 64:
            print("--batch must be in [1, 64]", file=sys.stderr)
            return 2
        return main_batched(args, lab)
    if args.weights == "w8g32" and args.exec_mode != "persistent":
        print("--weights w8g32 runs on the persistent decode only", file=sys.stderr)
        return 2
    if not 1 <= args.prompt or args.prompt + max(args.steps, args.warmup) + 1 > CAPACITY:
        print(f"--prompt plus the decoded tokens must fit the {CAPACITY}-position KV cache", file=sys.stderr)
        return 2
    prompt = [int(t) for t in lab.rng.uniform_ints(0, "bench.prompt", args.prompt, 16)]
    ms, wall, status, ck = run_decode(args, lab, prompt)
    if status:
        print(f"decode status 0x{status:x}", file=sys.stderr)
        return 1
    steps = args.steps
    ctx0 = args.prompt + 1
    kv = sum(KV_BYTES_PER_POSITION * (ctx0 + i) for i in range(steps))
    w8 = args.weights == "w8g32"
    algo = steps * ((W8_WEIGHT_BYTES + W8_EMBED_ROW_BYTES) if w8 else (WEIGHT_BYTES + EMBED_ROW_BYTES)) + kv
    achieved = algo / (ms * 1e-3) / 1e9
    per_token = None if w8 else traffic_from_profile()
    line = {
        "metric": W8_METRIC if w8 else METRIC,
        "value": round(steps / (ms * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x bf16 activations, fp32 accumulate" if w8 else "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, uniform prompt ids, seed 0)"
                + ("; weights quantized to w8g32 on the host" if w8 else ""),
        "config": {"workload": f"LFM2.5-230M-shape greedy decode, batch 1, {args.prompt}-token "
                               f"prompt then {steps} tokens ({args.exec_mode}"
                               + (", w8g32 weights)" if w8 else ")"),
                   "batch": 1, "prompt": args.prompt, "decode_tokens": steps,
                   "exec": args.exec_mode, "weights": args.weights},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     # the counter profile was taken on the default prompt
                     "traffic": None if per_token is None or args.prompt != PROMPT else round(per_token * steps)},
        "wall_ms": round(wall * 1e3, 3),
    }
    if not args.no_cpu and args.prompt <= 256 and not w8:
        line["cpu_baseline"] = cpu_baseline(prompt, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    # A successful run returns from the script normally: leaving through
    # sys.exit() has made rocprofv3 crash before writing its results for
    # processes that used cooperative launches.
    rc = main()
    if rc:
        sys.exit(rc)
