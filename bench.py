#!/usr/bin/env python
"""CyFA-400M bf16 on one MI355X: prefill tok/s (B=8, T=2048) and decode tok/s (B=64).

Workload (BASELINE.json metric; configs 3 and 4):
  prefill  CyFA-400M forward over B=8 x T=2048 uniform random token ids with
           use_cache=True (full logits, as the reference's model forward);
           one step = one prefill pass.  value = total prefill tokens / second.
  decode   B=64: a 2048-token prompt processed chunkwise (untimed), then
           greedy decode steps with the fused constant-memory decode kernel,
           each step one replay of the HIP-graph captured 24-layer step
           (argmax on the device). Reported under "decode".
Weights are seeded N(0, 0.02) random init (no checkpoints offline).

roofline: HIP events around every prefill attention launch in the timed
prefill region (cyfa_chunk_fwd_normed: the op with the layer's gated output
norm in its last kernel) give its average device duration; the decode kernel's duration comes
from HIP events around replays of a graph of in-place launches at the decode
shape (B=64, H=4), free of host launch gaps;
  prefill attention: 377 088 algorithmic FLOP per token*head / duration vs the
                     2.5 PFLOP/s dense bf16 MFMA peak, and (roofline.hbm) 2 572
                     algorithmic bytes per token*head (q, k, v, o, the output
                     norm's gate in bf16, three f32 gates) vs 8 TB/s;
  decode:            524 288 bytes of fp32 state per (batch, head) per launch of
                     cyfa_decode_layer_step, the kernel of the model's graphed
                     decode step, vs 8 TB/s (decode.op_kernel: the same for
                     cyfa_decode_step, fused_recurrent_cyfa alone).
isolated_pass: configuration 2 (B=8, H=4, T=4096), one scalar_la pass at each
pass shape ((K, V) = (256, 128) and (128, 256)), q, k, v ~ N(0, 1) bf16 with q, k
L2-normalised, log alpha = logsigmoid(N(3, 1)); HIP events around each launch;
156 032 FLOP per token*head per pass against the bf16 MFMA peak and the
algorithmic bytes (q, k, v, g in, o out) against 8 TB/s.
long_context: configuration 5 (CyFA-1.4B, B=1, a 16384-token prefill, 512
greedy decode steps) with the op's and the decode layer kernel's fractions.
measured_peaks: the box's achievable rates measured in the same run (a bf16
8192^3 GEMM through hipBLASLt and a 1 GiB device copy); each roofline also
gives its fraction of them (frac_of_measured) beside the vendor-peak frac.
backward: the chunk op's backward pass (cyfa_chunk_bwd: fp32 recompute and
adjoints) at configuration 3's attention shape (B=8, T=2048, H=4, K=V=256,
128 slots) with bf16 q, k, v and a bf16 cotangent of o; HIP events around each
launch, next to the forward launch's duration.
cpu_baseline: the CPU oracle (the restatement of the reference path; the
reference itself has no CPU path) timed on this host, bounded sample, median
of three after a warm-up, with the GPU's logits of the same sequence compared
against the oracle's.
"""

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "cyfa-jittor_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
FLOP_PER_TOKEN_HEAD = 377_088      # pass 1 + readout + pass 2, causal-exact
STATE_BYTES_PER_BH = 524_288       # fp32 hk + hv, read and written, K = V = 256
FLOP_PER_TOKEN_HEAD_PASS = 156_032  # one ScalarGatedLA pass, causal-exact
# Algorithmic HBM bytes of the prefill op per token*head: q, k, v and o in bf16
# (4 x 512) and the three f32 gates (12), plus the gated output norm's bf16 gate
# input (512) that the model's normed launch reads.
BYTES_PER_TOKEN_HEAD = 2 * 256 * 4 + 12 + 2 * 256
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE,
# scaled by a 1 GiB copy kernel (profiles/cyfa_chunk_fwd_cfg3_prefill.md,
# profiles/cyfa_decode_step_cfg4.md); they apply to the default shapes.
TRAFFIC_PREFILL_BYTES = 337.0e6    # one cyfa_chunk_fwd_normed at B=8, T=2048, H=4 (248.3 MB read + 88.7 MB written)
TRAFFIC_DECODE_BYTES = 135.5e6     # one decode launch at B=64, H=4
TRAFFIC_LAYER_STEP_BYTES = 138.1e6  # one cyfa_decode_layer_step at B=64, H=4 (69.6 MB read + 68.5 MB written)


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10, help="timed prefill steps")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--decode-warmup", type=int, default=4)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq-len", type=int, default=2048)
    ap.add_argument("--decode-batch", type=int, default=64)
    ap.add_argument("--config", default="cyclic_flow_attention_400m.json")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-isolated", action="store_true", help="skip the configuration-2 scalar_la timings")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip configuration 5: CyFA-1.4B, B=1, a 16384-token prefill, then 512 greedy "
                         "decode steps (reported under 'long_context')")
    ap.add_argument("--no-backward", action="store_true", help="skip the op's backward-pass timing")
    ap.add_argument("--no-measured-peaks", action="store_true",
                    help="skip the bf16 GEMM and copy measurements of the box's achievable rates")
    ap.add_argument("--decode-kernel-only", action="store_true",
                    help="only time the fused decode kernel at the decode shape (for hardware-counter runs)")
    ap.add_argument("--layer-kernel-only", action="store_true",
                    help="only run the decode layer-step kernel at the decode shape, eagerly (for hardware-counter runs)")
    ap.add_argument("--no-tuned-gemms", action="store_true",
                    help="leave the library GEMMs on their default solutions")
    ap.add_argument("--tune-gemms", metavar="FILE",
                    help="time the GEMM solutions of every shape this run executes and write the "
                         "selections to FILE (TunableOp results; see cyclic_flow_attention/gemm_tuning.py)")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="run one fp32 copy kernel (out = 1.0 * in) of this many MiB before the prefill, "
                         "as the known-size reference for HBM byte counters")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads():
    """Threads of the CPU baseline: every core of the affinity set, capped at
    16, the host share of one GPU on the MI355X boxes (whose affinity set
    shows every core of the host)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_cores_visible():
    return len(os.sched_getaffinity(0))


def decode_step_bytes(model, batch):
    """HBM bytes one greedy decode step must move at least: every weight once
    (the embedding table only for the batch's rows), the fp32 recurrent states
    read and written, the conv caches read and written."""
    import torch

    cfg = model.config
    weights = sum(p.numel() * p.element_size() for n, p in model.named_parameters() if "embeddings" not in n)
    weights += batch * cfg.hidden_size * model.model.embeddings.weight.element_size()
    layers = cfg.num_hidden_layers
    H = cfg.num_heads
    state = STATE_BYTES_PER_BH * batch * H * layers
    conv = 2 * batch * (cfg.conv_size - 1) * 3 * H * 256 * 2 * layers
    return weights, state + conv


def build_model(cfg_name, device):
    import torch

    from cyclic_flow_attention.utils import initialize_model, read_config

    config = read_config(cfg_name)
    model = initialize_model(config, std=0.02, seed=0).to(device).eval()
    return config, model


def time_prefill(model, ids, steps, warmup):
    import torch

    from cyclic_flow_attention import _native

    with torch.no_grad():
        for _ in range(warmup):
            model(ids, use_cache=True)
        torch.cuda.synchronize()
        with _native.LaunchTimer() as timer:
            start = time.perf_counter()
            for _ in range(steps):
                out = model(ids, use_cache=True)
            torch.cuda.synchronize()
            elapsed = time.perf_counter() - start
        first_row = out["logits"][0].float().cpu()
        del out
    res = timer.results()
    return elapsed, res.get("cyfa_chunk_fwd_normed", []) + res.get("cyfa_chunk_fwd", []), first_row


def time_isolated_pass(K, V, B=8, H=4, T=4096, reps=20, warmup=3):
    """Average device duration (ms) of one scalar_la launch at configuration 2."""
    import torch

    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops.chunk import scalar_la

    gen = torch.Generator(device="cuda").manual_seed(2)
    q = torch.nn.functional.normalize(torch.randn(B, H, T, K, device="cuda", generator=gen), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(B, H, T, K, device="cuda", generator=gen), dim=-1).bfloat16()
    v = torch.randn(B, H, T, V, device="cuda", generator=gen).bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, T, device="cuda", generator=gen) + 3)
    raw = K == 256  # the pass-1 shape returns the raw fp32 sum of the slices
    scale = K ** -0.5 if K == 256 else 1.0
    with torch.no_grad():
        for _ in range(warmup):
            scalar_la(q, k, v, g, None, scale, raw)
        torch.cuda.synchronize()
        with _native.LaunchTimer() as timer:
            for _ in range(reps):
                scalar_la(q, k, v, g, None, scale, raw)
            ms = timer.results().get("cyfa_scalar_la", [])
    per_th = 2 * K + 2 * K + 2 * V + 4 + (4 if raw else 2) * V  # q, k, v, g read; o written
    return statistics.fmean(ms), per_th * B * H * T, FLOP_PER_TOKEN_HEAD_PASS * B * H * T


def time_backward(B=8, T=2048, H=4, reps=5, warmup=2):
    """Average device durations (ms) of the chunk op's forward and backward
    launches at configuration 3's attention shape."""
    import torch

    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops import chunk_cyfa

    gen = torch.Generator(device="cuda").manual_seed(3)
    K = V = 256
    x = dict(
        q=torch.randn(B, T, H, K, device="cuda", generator=gen).bfloat16(),
        k=torch.randn(B, T, H, K, device="cuda", generator=gen).bfloat16(),
        v=torch.randn(B, T, H, V, device="cuda", generator=gen).bfloat16(),
        g=torch.nn.functional.logsigmoid(torch.randn(B, T, H, device="cuda", generator=gen) + 3),
        delta=torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=gen)),
        beta=torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=gen)),
        readout=torch.eye(127, device="cuda").expand(H, 127, 127).contiguous(),
        q_norm_weight=torch.ones(K, device="cuda"),
        k_norm_weight=torch.ones(K, device="cuda"),
    )
    leaves = [t.requires_grad_(True) for t in x.values()]
    d_o = torch.randn(B, T, H, V, device="cuda", generator=gen).bfloat16()
    for _ in range(warmup):
        o, _ = chunk_cyfa(**x)
        torch.autograd.grad(o, leaves, d_o)
    torch.cuda.synchronize()
    with _native.LaunchTimer() as timer:
        for _ in range(reps):
            o, _ = chunk_cyfa(**x)
            torch.autograd.grad(o, leaves, d_o)
        res = timer.results()
    return statistics.fmean(res["cyfa_chunk_fwd"]), statistics.fmean(res["cyfa_chunk_bwd"])


def measured_peaks(reps=10):
    """The box's achievable rates, measured next to the results: a bf16 GEMM
    of 8192 x 8192 x 8192 through the library (hipBLASLt, matrix cores) and a
    device-to-device copy of 1 GiB (read + write), each the median of reps."""
    import torch

    a = torch.randn(8192, 8192, device="cuda").bfloat16()
    b = torch.randn(8192, 8192, device="cuda").bfloat16()
    src = torch.empty(1 << 28, device="cuda")  # 1 GiB of fp32
    dst = torch.empty_like(src)

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        ms = []
        for _ in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            fn()
            end.record()
            end.synchronize()
            ms.append(start.elapsed_time(end))
        return statistics.median(ms)

    gemm_ms = timed(lambda: torch.matmul(a, b))
    copy_ms = timed(lambda: dst.copy_(src))
    del a, b, src, dst
    torch.cuda.empty_cache()
    return {
        "bf16_gemm": {"achieved": round(2 * 8192 ** 3 / (gemm_ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s",
                      "what": "torch.matmul bf16 8192 x 8192 x 8192 (hipBLASLt), median of 10"},
        "hbm_copy": {"achieved": round(2 * (1 << 30) / (copy_ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                     "what": "device copy of 1 GiB fp32 (read + write bytes), median of 10"},
    }


def time_decode(model, prompt, steps, warmup):
    """Greedy decode after a chunkwise prompt; one step = one replay of the
    HIP-graph captured 24-layer decode step (argmax on the device)."""
    import torch

    with torch.no_grad():
        hidden, cache = model.model(prompt, use_cache=True)
        tok = model.lm_head(hidden[:, -1:]).argmax(-1)
        del hidden
        dec = model.graphed_decoder(cache, tok)
        del cache
        for _ in range(warmup):
            dec.step()
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(steps):
            dec.step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start
    return elapsed


def decode_layer_kernel_ms(batch, heads, reps=24, replays=5, graphed=True, gate_in_kernel=None):
    """Average device time of one cyfa_decode_layer_step launch (the kernel the
    model's graphed decode step runs: short convolution, gates, the decode op
    and the gated output norm) at the decode shape, timed as decode_kernel_ms:
    `reps` in-place launches on their own states captured in one graph,
    replayed between HIP events on the launch stream. gate_in_kernel: the
    kernel also forms the gate (g_proj[1]) from g0, as the model's step does
    at GATE_IN_KERNEL_MIN_WORKGROUPS or more (batch, head) workgroups; None
    picks the model's choice for this shape."""
    import torch

    from cyclic_flow_attention import _native
    from cyclic_flow_attention.layers.cyfa import GATE_IN_KERNEL_MIN_WORKGROUPS
    from cyclic_flow_attention.ops.fused_recurrent import decode_layer_step

    if gate_in_kernel is None:
        gate_in_kernel = batch * heads >= GATE_IN_KERNEL_MIN_WORKGROUPS

    dev = torch.device("cuda:0")
    H, D = heads, 3 * heads * 256
    gen = torch.Generator().manual_seed(6)
    qkv = torch.randn(batch, 1, D, generator=gen).bfloat16().to(dev)
    wconv = (0.3 * torch.randn(D, 4, generator=gen)).bfloat16().to(dev)
    abd = torch.randn(batch, 1, 3 * H, generator=gen).bfloat16().to(dev)
    dt_bias, A_log = torch.randn(H, generator=gen).to(dev), torch.randn(H, generator=gen).to(dev)
    gate = torch.randn(batch, 1, H * 256, generator=gen).bfloat16().to(dev)
    g_proj = None
    if gate_in_kernel:
        g_proj = (torch.randn(batch, 1, 256, generator=gen).bfloat16().to(dev),
                  (0.06 * torch.randn(H * 256, 256, generator=gen)).bfloat16().to(dev),
                  (0.5 * torch.randn(H * 256, generator=gen)).bfloat16().to(dev))
        gate = None
    ones = torch.ones(256, device=dev)
    table = _native.readout_table(torch.eye(127, device=dev).expand(H, 127, 127).contiguous())
    states = [(torch.randn(batch, heads, 256, 128, device=dev), torch.randn(batch, heads, 128, 256, device=dev),
               torch.rand(batch, heads, device=dev),
               (0.5 * torch.randn(batch, 3, D, device=dev)).bfloat16()) for _ in range(reps)]

    def step(st):
        decode_layer_step(qkv, st[3], st[3], wconv, abd, dt_bias, A_log, gate, ones, 1e-6, 127.0, table, ones, ones,
                          1e-6, 1e-6, H, initial_state=st[:3], output_final_state=True, inplace=True, g_proj=g_proj)

    with torch.no_grad():
        step(states[0])
        torch.cuda.synchronize()
        if not graphed:  # one eager launch per state (hardware-counter runs attach per dispatch)
            for st in states:
                step(st)
            torch.cuda.synchronize()
            return None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for st in states:
                step(st)
        graph.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(replays):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * replays)


def decode_kernel_ms(batch, heads, reps=24, replays=5, graphed=True):
    """Average device time of one fused decode launch at the decode shape.

    `reps` in-place launches, each on its own state (one per layer of the
    400M model: 24 x 134 MB, far beyond the 256 MB last-level cache, so every
    launch streams its state from HBM as in the model's decode step), are
    captured in one HIP graph and the graph is replayed between two HIP events
    on the launch stream, so host launch gaps do not enter the figure."""
    import torch

    from cyclic_flow_attention.ops import fused_recurrent_cyfa
    from cyclic_flow_attention.ops.utils import readout_table

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(5)
    x = dict(q=torch.randn(batch, 1, heads, 256, generator=gen).bfloat16(),
             k=torch.randn(batch, 1, heads, 256, generator=gen).bfloat16(),
             v=torch.randn(batch, 1, heads, 256, generator=gen).bfloat16(),
             g=torch.nn.functional.logsigmoid(torch.randn(batch, 1, heads, generator=gen) + 3),
             delta=torch.sigmoid(torch.randn(batch, 1, heads, generator=gen)),
             beta=torch.sigmoid(torch.randn(batch, 1, heads, generator=gen)),
             readout=torch.eye(127).expand(heads, 127, 127).clone(),
             q_norm_weight=torch.ones(256), k_norm_weight=torch.ones(256))
    x = {k: v.to(dev) for k, v in x.items()}
    table = readout_table(x["readout"])
    states = [(torch.randn(batch, heads, 256, 128, device=dev), torch.randn(batch, heads, 128, 256, device=dev),
               torch.rand(batch, heads, device=dev)) for _ in range(reps)]
    with torch.no_grad():
        fused_recurrent_cyfa(**x, initial_state=states[0], output_final_state=True, table=table, inplace=True)
        torch.cuda.synchronize()
        if not graphed:  # eager launches, one dispatch each (hardware-counter runs)
            for st in states:
                fused_recurrent_cyfa(**x, initial_state=st, output_final_state=True, table=table, inplace=True)
            torch.cuda.synchronize()
            return None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for st in states:
                fused_recurrent_cyfa(**x, initial_state=st, output_final_state=True, table=table, inplace=True)
        graph.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(replays):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * replays)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_prefill(model, config, seq_len, gpu_logits=None, reps=3):
    """Oracle forward (float32, reference rounding points) of one whole
    sequence of the prefill batch on the host cores: the median of `reps`
    timed forwards after a warm-up forward. With the GPU's logits of the same
    sequence (gpu_logits [T, V]), also reports how far they are from the
    oracle's."""
    import torch

    from oracle import model_oracle

    threads = cpu_threads()
    torch.set_num_threads(threads)
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = {k: getattr(config, k) for k in config.__dataclass_fields__}
    gen = torch.Generator().manual_seed(0)  # the prefill batch's ids: its first row
    ids = torch.randint(0, config.vocab_size, (1, seq_len), generator=gen)
    times = []
    with torch.no_grad():
        model_oracle.causal_lm(params, cfg, ids[:, :256], mode="mirror")  # warm-up
        for _ in range(reps):
            start = time.perf_counter()
            logits, _ = model_oracle.causal_lm(params, cfg, ids, use_cache=True, mode="mirror")
            times.append(time.perf_counter() - start)
    elapsed = statistics.median(times)
    out = {
        "value": round(seq_len / elapsed, 2),
        "unit": "tok/s",
        "cores": threads,
        "cores_visible": cpu_cores_visible(),
        "kind": "port",
        "cpu": cpu_model(),
        "sample": f"CPU oracle (float32, bf16 rounding points) full 400M forward of the prefill batch's first "
                  f"sequence, B=1 x T={seq_len}: median of {reps} after a warm-up, {elapsed:.2f} s",
    }
    if gpu_logits is not None:
        a = gpu_logits.double().cpu()
        b = logits[0].double()
        diff = (a - b).abs()
        out["parity"] = {"what": "GPU logits of that sequence vs the oracle's (mirror mode)",
                         "max_abs": round(diff.max().item(), 4),
                         "mean_rel": round((diff.mean() / b.abs().mean()).item(), 5),
                         "top1_agree": round((a.argmax(-1) == b.argmax(-1)).double().mean().item(), 4)}
    return out


def cpu_baseline_decode(model, config, batch, steps=4, reps=3):
    """Oracle decode steps on the host at the decode batch, from the state of
    a short oracle prefill (the per-step work does not depend on the prompt
    length): the median over `reps` runs of `steps` steps, after a warm-up step."""
    import torch

    from oracle import model_oracle

    threads = cpu_threads()
    torch.set_num_threads(threads)
    params = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = {k: getattr(config, k) for k in config.__dataclass_fields__}
    gen = torch.Generator().manual_seed(2)
    ids = torch.randint(0, config.vocab_size, (batch, 64), generator=gen)
    times = []
    with torch.no_grad():
        logits, cache = model_oracle.causal_lm(params, cfg, ids, use_cache=True, mode="mirror")
        tok = logits[:, -1].argmax(-1, keepdim=True)
        logits, cache = model_oracle.causal_lm(params, cfg, tok, cache=cache, use_cache=True, mode="mirror")  # warm-up
        for _ in range(reps):
            start = time.perf_counter()
            for _ in range(steps):
                logits, cache = model_oracle.causal_lm(params, cfg, tok, cache=cache, use_cache=True, mode="mirror")
                tok = logits[:, -1].argmax(-1, keepdim=True)
            times.append(time.perf_counter() - start)
    elapsed = statistics.median(times)
    return {
        "value": round(batch * steps / elapsed, 2),
        "unit": "tok/s",
        "cores": threads,
        "cores_visible": cpu_cores_visible(),
        "kind": "port",
        "cpu": cpu_model(),
        "sample": f"CPU oracle (float32) decode of the 400M model at B={batch} after a 64-token prompt: median of "
                  f"{reps} runs of {steps} steps after a warm-up step, {elapsed:.2f} s per run",
    }


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU: the CyFA hot path shards over (batch, head) "
                                   "with no exchange inside the op; run with --gpus 1"}), flush=True)
        return 2

    import torch

    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.decode_kernel_only:
        decode_kernel_ms(args.decode_batch, 4, graphed=False)
        log(f"decode kernel: 24 launches at B={args.decode_batch}, H=4, one state each")
        return 0
    if args.layer_kernel_only:
        decode_layer_kernel_ms(args.decode_batch, 4, graphed=False)
        log(f"decode layer-step kernel: 25 launches at B={args.decode_batch}, H=4, one state each")
        return 0
    log(f"device {torch.cuda.get_device_name(dev)}")
    from cyclic_flow_attention import gemm_tuning

    if args.tune_gemms:
        gemm_tuning.tune_gemms(args.tune_gemms)
        log(f"GEMM solutions: tuning, selections to {args.tune_gemms}")
    elif not args.no_tuned_gemms:
        used = gemm_tuning.use_tuned_gemms()
        log(f"GEMM solutions: {'TunableOp selections ' + str(gemm_tuning.DEFAULT_FILE.name) if used else 'library defaults'}")
    config, model = build_model(args.config, dev)
    H = config.num_heads
    gen = torch.Generator().manual_seed(0)
    ids = torch.randint(0, config.vocab_size, (args.batch, args.seq_len), generator=gen).to(dev)

    if args.calibration_copy_mib:
        n = args.calibration_copy_mib * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calibration_copy_mib} MiB read + {args.calibration_copy_mib} MiB written")
        del src, dst

    log(f"prefill B={args.batch} T={args.seq_len}: warmup {args.warmup}, timed {args.steps}")
    elapsed, op_ms, first_row_logits = time_prefill(model, ids, args.steps, args.warmup)
    tokens = args.batch * args.seq_len * args.steps
    value = tokens / elapsed
    op_avg = statistics.fmean(op_ms) if op_ms else float("nan")
    flop = FLOP_PER_TOKEN_HEAD * args.batch * args.seq_len * H
    achieved = flop / (op_avg * 1e-3) / 1e12
    op_bytes = BYTES_PER_TOKEN_HEAD * args.batch * args.seq_len * H
    op_gbs = op_bytes / (op_avg * 1e-3) / 1e9
    log(f"prefill {value:,.0f} tok/s; attention op {op_avg:.3f} ms/launch over {len(op_ms)} launches "
        f"= {achieved:.1f} TFLOP/s, {op_gbs:,.0f} GB/s algorithmic")
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: uniform random token ids; seeded N(0, 0.02) random-init CyFA-400M weights",
        "config": {
            "workload": f"CyFA-400M prefill B={args.batch} x T={args.seq_len} (config 3) as value; "
                        f"decode B={args.decode_batch} after a {args.seq_len}-token prompt (config 4) under 'decode'",
            "global_batch": args.batch,
            "seq_len": args.seq_len,
            "parallelism": "single-gpu",
        },
        "roofline": {
            "kernel": "cyfa_chunk_fwd_normed (segment states, pass 1 with the slot readout, "
                      "pass 2 with the gated output norm); FLOP of the attention op only",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": TRAFFIC_PREFILL_BYTES if (args.batch, args.seq_len, H) == (8, 2048, 4) else None,
            "launch_ms": round(op_avg, 4),
            "flop_per_launch": flop,
            "hbm": {"achieved": round(op_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(op_gbs / PEAK_HBM_GBS, 4), "algorithmic_bytes": op_bytes},
        },
    }

    if not args.no_decode:
        prompt = torch.randint(0, config.vocab_size, (args.decode_batch, args.seq_len), generator=gen).to(dev)
        log(f"decode B={args.decode_batch}: prompt {args.seq_len}, warmup {args.decode_warmup}, "
            f"timed {args.decode_steps}")
        d_elapsed = time_decode(model, prompt, args.decode_steps, args.decode_warmup)
        d_value = args.decode_batch * args.decode_steps / d_elapsed
        d_bytes = STATE_BYTES_PER_BH * args.decode_batch * H
        l_bytes = d_bytes
        # the kernel in the form the model's step runs it (g_proj[1] inside at
        # this shape), then with a precomputed gate, then the op alone
        l_avg = decode_layer_kernel_ms(args.decode_batch, H)
        l_gbs = l_bytes / (l_avg * 1e-3) / 1e9
        lp_avg = decode_layer_kernel_ms(args.decode_batch, H, gate_in_kernel=False)
        lp_gbs = l_bytes / (lp_avg * 1e-3) / 1e9
        d_avg = decode_kernel_ms(args.decode_batch, H)
        d_gbs = d_bytes / (d_avg * 1e-3) / 1e9
        from cyclic_flow_attention.layers.cyfa import GATE_IN_KERNEL_MIN_WORKGROUPS

        in_kernel = args.decode_batch * H >= GATE_IN_KERNEL_MIN_WORKGROUPS
        w_bytes, s_bytes = decode_step_bytes(model, args.decode_batch)
        step_ms = d_elapsed / args.decode_steps * 1e3
        step_gbs = (w_bytes + s_bytes) / (step_ms * 1e-3) / 1e9
        log(f"decode {d_value:,.0f} tok/s ({step_gbs:,.0f} GB/s of weights + states); layer-step kernel "
            f"{l_avg * 1e3:.1f} us/launch = {l_gbs:,.0f} GB/s (gate precomputed {lp_avg * 1e3:.1f} us); "
            f"op kernel {d_avg * 1e3:.1f} us/launch = {d_gbs:,.0f} GB/s")
        result["decode"] = {
            "value": round(d_value, 1),
            "unit": "tok/s",
            "batch": args.decode_batch,
            "steps": args.decode_steps,
            "ms_per_step": round(step_ms, 3),
            "roofline": {
                "kernel": "cyfa_decode_layer_step as the model's graphed step runs it at this shape (short conv, "
                          "gates, decode op, gated output norm" + (", g_proj[1] formed inside)" if in_kernel else ")"),
                "bound": "hbm",
                "achieved": round(l_gbs, 1),
                "peak": PEAK_HBM_GBS,
                "unit": "GB/s",
                "frac": round(l_gbs / PEAK_HBM_GBS, 4),
                "traffic": TRAFFIC_LAYER_STEP_BYTES if (args.decode_batch, H) == (64, 4) else None,
                "launch_us": round(l_avg * 1e3, 2),
                "bytes_per_launch": l_bytes,
            },
            "layer_kernel_gate_precomputed": {
                "kernel": "cyfa_decode_layer_step with g_proj[1] precomputed",
                "achieved": round(lp_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(lp_gbs / PEAK_HBM_GBS, 4), "launch_us": round(lp_avg * 1e3, 2),
            },
            "op_kernel": {
                "kernel": "cyfa_decode_step (fused_recurrent_cyfa alone)",
                "achieved": round(d_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(d_gbs / PEAK_HBM_GBS, 4),
                "traffic": TRAFFIC_DECODE_BYTES if (args.decode_batch, H) == (64, 4) else None,
                "launch_us": round(d_avg * 1e3, 2),
            },
            "step_roofline": {
                "what": "whole graphed decode step: every weight once (embedding rows only) plus the fp32 states and "
                        "conv caches read and written, per step time",
                "bound": "hbm", "achieved": round(step_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(step_gbs / PEAK_HBM_GBS, 4),
                "weight_bytes": w_bytes, "state_bytes": s_bytes,
            },
        }
        del prompt

    if not args.no_measured_peaks:
        peaks = measured_peaks()
        gemm, copy = peaks["bf16_gemm"]["achieved"], peaks["hbm_copy"]["achieved"]
        result["measured_peaks"] = peaks
        result["roofline"]["frac_of_measured"] = round(achieved / gemm, 4)
        result["roofline"]["hbm"]["frac_of_measured"] = round(op_gbs / copy, 4)
        if "decode" in result:
            result["decode"]["roofline"]["frac_of_measured"] = round(result["decode"]["roofline"]["achieved"] / copy, 4)
        log(f"measured peaks: bf16 GEMM {gemm:,.1f} TFLOP/s, copy {copy:,.0f} GB/s")

    if not args.no_isolated:
        iso = {"workload": "scalar_la, configuration 2: B=8, H=4, T=4096, zero initial state"}
        for name, (K, V) in (("pass1_shape", (256, 128)), ("pass2_shape", (128, 256))):
            ms, nbytes, flop = time_isolated_pass(K, V)
            tflops = flop / (ms * 1e-3) / 1e12
            gbs = nbytes / (ms * 1e-3) / 1e9
            iso[name] = {
                "K": K, "V": V, "launch_us": round(ms * 1e3, 2),
                "mfma": {"achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / PEAK_BF16_TFLOPS, 4)},
                "hbm": {"achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "algorithmic_bytes": nbytes},
            }
            log(f"scalar_la K={K} V={V}: {ms * 1e3:.1f} us/launch = {tflops:.1f} TFLOP/s, {gbs:,.0f} GB/s algorithmic")
        result["isolated_pass"] = iso

    if not args.no_backward:
        fwd_ms, bwd_ms = time_backward()
        result["backward"] = {
            "workload": "cyfa_chunk_bwd at configuration 3's attention shape: B=8, T=2048, H=4, K=V=256, 128 slots, "
                        "bf16 q, k, v and cotangent; gradients of q, k, v, g, delta, beta, readout, norm weights",
            "launch_ms": round(bwd_ms, 3), "forward_launch_ms": round(fwd_ms, 4),
            "train_tok_per_s": round(8 * 2048 / ((fwd_ms + bwd_ms) * 1e-3), 1),
        }
        log(f"backward: {bwd_ms:.3f} ms per launch (forward {fwd_ms * 1e3:.1f} us)")

    if not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline_prefill(model, config, args.seq_len, first_row_logits)
        log(f"cpu prefill {result['cpu_baseline']['value']} tok/s")
        if "decode" in result:
            result["decode"]["cpu_baseline"] = cpu_baseline_decode(model, config, args.decode_batch)
            log(f"cpu decode {result['decode']['cpu_baseline']['value']} tok/s")

    if not args.no_long_context:
        del model
        torch.cuda.empty_cache()
        lc_config, lc_model = build_model("cyclic_flow_attention_1_4b.json", dev)
        T5, H5 = 16384, lc_config.num_heads
        lc_ids = torch.randint(0, lc_config.vocab_size, (1, T5), generator=gen).to(dev)
        log(f"long context: CyFA-1.4B prefill B=1 T={T5}")
        lc_elapsed, lc_op_ms, _ = time_prefill(lc_model, lc_ids, 2, 1)
        lc_op = statistics.fmean(lc_op_ms)
        lc_flop = FLOP_PER_TOKEN_HEAD * T5 * H5
        lc_bytes = BYTES_PER_TOKEN_HEAD * T5 * H5
        log(f"long context: decode B=1, 512 steps after the {T5}-token prompt")
        lc_dec = time_decode(lc_model, lc_ids, 512, 4)
        lc_kernel = decode_layer_kernel_ms(1, H5)
        lc_state = STATE_BYTES_PER_BH * H5
        lc_w, lc_s = decode_step_bytes(lc_model, 1)
        lc_step_gbs = (lc_w + lc_s) / (lc_dec / 512) / 1e9
        result["long_context"] = {
            "workload": f"configuration 5: CyFA-1.4B, B=1, {T5}-token prefill, then 512 greedy decode steps",
            "prefill": {"value": round(2 * T5 / lc_elapsed, 1), "unit": "tok/s",
                        "ms_per_step": round(lc_elapsed / 2 * 1e3, 3),
                        "op_launch_ms": round(lc_op, 4),
                        "mfma_frac": round(lc_flop / (lc_op * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                        "hbm_frac": round(lc_bytes / (lc_op * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
            "decode": {"value": round(512 / lc_dec, 1), "unit": "tok/s", "ms_per_step": round(lc_dec / 512 * 1e3, 4),
                       "step_roofline": {
                           "what": "whole graphed B=1 step: every weight once plus the fp32 states and conv caches "
                                   "read and written, per step time",
                           "bound": "hbm", "achieved": round(lc_step_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(lc_step_gbs / PEAK_HBM_GBS, 4), "weight_bytes": lc_w, "state_bytes": lc_s},
                       "layer_kernel_us": round(lc_kernel * 1e3, 2),
                       "layer_kernel_state_hbm_frac": round(lc_state / (lc_kernel * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        }
        log(f"long context: prefill {2 * T5 / lc_elapsed:,.0f} tok/s (op {lc_op * 1e3:.1f} us), decode "
            f"{512 / lc_dec:,.1f} tok/s (layer kernel {lc_kernel * 1e3:.1f} us)")
        del lc_model

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
