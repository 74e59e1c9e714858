"""WKV7 benchmark on one MI355X: prefill and T=1 decode
(config 2), synthetic seeded inputs resident in HBM.

A step is one call of the packed fp32-state recurrence
(``_C.tmix_wkv7_recurrent_fp32_from_decay_logits`` with a reused metadata
ticket, as benchmarks/tmix/wkv7/bench.py:309-365 of the reference does) over
the whole batch.  W warm-up steps, then K timed steps between a
synchronize/event pair; the state pool is reset before the timed region.
tokens/s = total tokens per step / seconds per step.

``roofline`` is measured live: the dominant kernel is launched K more times
through the C ABI directly (no Python checks between launches) on the same
torch stream, bracketed by HIP events, and its algorithmic bytes
(896 B per token-head + 2 x 16 KiB of fp32 state per sequence-head) are
divided by the average launch duration.

``cpu_baseline`` times the oracle's fp32 C recurrence (OpenMP over
sequence x head) on the host on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "WKV7 tokens/s at h32d64 bf16 (prefill + T=1 decode); % of HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
BYTES_PER_TOKEN_HEAD = 896          # 6 bf16 inputs x 64 + bf16 output x 64
STATE_BYTES = 64 * 64 * 4           # one fp32 64x64 state
MFMA_PEAK_TFLOPS = 2500.0           # dense bf16
# v_mfma_f32_16x16x32_bf16 instructions the ring chunked kernel issues per
# 16-token chunk of one head: 30 token-token products (5 products x 3 split
# terms x 2 key halves) + 16 for T on the key side, 4 x 30 on the state side
# (bf16 hi/lo split products); rocprofv3 SQ_INSTS_MFMA reads 166 x 65 536
# chunks per config-1 dispatch
MFMA_PER_CHUNK = 166
MFMA_FLOPS = 16 * 16 * 32 * 2


def algorithmic_bytes(total_tokens: int, heads: int, sequences: int) -> int:
    return total_tokens * heads * BYTES_PER_TOKEN_HEAD + 2 * sequences * heads * STATE_BYTES


class Runner:
    """One workload with its ticket, output buffer and a state pool."""

    def __init__(self, w, torch, flashrwkv2_amd):
        self.w = w
        self.torch = torch
        self.C = flashrwkv2_amd._C
        self.state0 = w.state_pool
        self.state = w.state_pool.clone()
        self.out = torch.empty_like(w.v)
        self.ticket = flashrwkv2_amd.prepare_tmix_wkv7_recurrent_metadata(
            w.cu_seqlens, w.state_indices, total_tokens=w.total_tokens,
            state_pool_size=w.state_pool.shape[0])
        from flashrwkv2_amd import _native as N

        self.N = N
        self.lib = N.load()
        t = self.ticket
        self._direct = (t._query_start_loc_snapshot().data_ptr(),
                        t._state_indices_snapshot().data_ptr(), t._status().data_ptr(),
                        w.state_indices.numel(), w.num_heads, 64, w.total_tokens,
                        t._max_seqlen(), N.FR2_DTYPE_BFLOAT16, self.state.data_ptr(),
                        w.r.data_ptr(), w.decay_logits.data_ptr(), None, w.k.data_ptr(),
                        w.v.data_ptr(), w.a.data_ptr(), w.b.data_ptr(), self.out.data_ptr(),
                        1.0)

    def step(self):
        w = self.w
        self.C.tmix_wkv7_recurrent_fp32_from_decay_logits(
            w.cu_seqlens, w.state_indices, self.state, *w.tokens, self.out, 1.0, None,
            self.ticket)

    def direct(self, stream_handle):
        rc = self.lib.fr2_wkv7_recurrent_fp32_forward(*self._direct, stream_handle)
        if rc:
            self.N.check(rc, "fr2_wkv7_recurrent_fp32_forward")

    def reset(self):
        self.state.copy_(self.state0)

    def time_steps(self, steps: int, warmup: int, settle_s: float = 0.0) -> float:
        """ms per public step over exactly `steps` timed steps, after `warmup`
        untimed steps and, with settle_s > 0, further untimed steps until
        settle_s seconds have passed since the warm-up began (the shader clock
        ramps up over the first tens of milliseconds of sustained work).  Each
        timed step is also bracketed by its own event pair (self.step_stats)."""
        torch = self.torch
        t_begin = time.perf_counter()
        for _ in range(warmup):
            self.step()
        torch.cuda.synchronize()
        extra = 0
        while time.perf_counter() - t_begin < settle_s:
            for _ in range(16):
                self.step()
            extra += 16
            torch.cuda.synchronize()
        self.settle = {"seconds": round(time.perf_counter() - t_begin, 3),
                       "extra_steps": extra, "target_s": settle_s}
        self.reset()
        torch.cuda.synchronize()
        # the timed region: exactly `steps` public steps between one event
        # pair (events between steps would add their own commands to it)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            self.step()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        event_ms = e0.elapsed_time(e1)
        # per-step spread from a second, untimed pass with an event pair
        # around every step
        self.reset()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record()
        for j in range(steps):
            self.step()
            ev[j + 1].record()
        torch.cuda.synchronize()
        per = sorted(ev[j].elapsed_time(ev[j + 1]) for j in range(steps))
        self.step_stats = {"event_ms_mean": round(event_ms / steps, 5),
                           "wall_ms_mean": round(wall * 1e3 / steps, 5),
                           "per_step_pass": {"event_ms_min": round(per[0], 5),
                                             "event_ms_median": round(per[len(per) // 2], 5),
                                             "event_ms_max": round(per[-1], 5)}}
        return max(event_ms, wall * 1e3) / steps

    def time_kernel(self, launches: int) -> float:
        """Average device duration of one launch (ms), direct C-ABI launches."""
        torch = self.torch
        stream = torch.cuda.current_stream()
        handle = stream.cuda_stream
        for _ in range(3):
            self.direct(handle)
        self.reset()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(launches):
            self.direct(handle)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / launches

    def kernel_name(self) -> str:
        """The kernel the library's policy picks for this launch, as the
        library reports it (fr2_wkv7_recurrent_fp32_dispatch)."""
        w = self.w
        return self.C.dispatch_kernel_name(w.state_indices.numel(), w.num_heads, 64,
                                           w.total_tokens, self.ticket._max_seqlen())


def cpu_baseline(w, threads: int, sample_tokens: int | None, min_seconds: float = 12.0):
    """fp32 C recurrence on the host over the first `sample_tokens` tokens of
    every sequence (all heads), repeated until `min_seconds` of CPU time."""
    import numpy as np

    import oracle

    cu = w.cu_seqlens.cpu().numpy()
    lens = np.diff(cu)
    take = lens if sample_tokens is None else np.minimum(lens, sample_tokens)
    idx = np.concatenate([np.arange(cu[i], cu[i] + take[i]) for i in range(len(lens))])
    toks = [t.float().cpu().numpy()[idx] for t in w.tokens]
    cu_s = np.concatenate([[0], np.cumsum(take)]).astype(np.int32)
    pool = w.state_pool.cpu().numpy()
    oracle.wkv7_cpu_f32(*(t[: cu_s[1]] for t in toks), cu_seqlens=cu_s[:2],
                        state_pool=pool[:1], threads=threads)  # warm-up
    n_tok = int(take.sum())
    reps, dt = 0, 0.0
    while dt < min_seconds:
        t0 = time.perf_counter()
        oracle.wkv7_cpu_f32(*toks, cu_seqlens=cu_s,
                            state_indices=np.arange(len(lens), dtype=np.int32),
                            state_pool=pool.copy(), threads=threads)
        dt += time.perf_counter() - t0
        reps += 1
    return n_tok * reps / dt, dt, n_tok, reps


def cpu_info() -> dict:
    """Host CPU of this run: logical CPUs, the ones this process may use, and
    the model name lscpu prints."""
    import subprocess

    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return {"nproc": os.cpu_count(), "usable": len(os.sched_getaffinity(0)), "model": model}


def cpu_baseline_plan(threads: int, repeats: int = 20) -> dict:
    """The planned pure-torch CPU baseline: the per-token fp32 loop
    (the form of the reference's test oracle, vectorised over heads) on config
    0 and on one config-2 decode step, median of `repeats` timed runs after a
    warm-up, with torch limited to `threads` threads."""
    import statistics

    import torch

    from flashrwkv2_amd import workloads
    from oracle.torch_loop import wkv7_torch_packed

    torch.set_num_threads(threads)
    legs = {}
    for name, w in (("cfg0_B1_T64_H4", workloads.config(0, "cpu", dtype=torch.float32)),
                    ("cfg2_decode_N256_H32_one_step", workloads.config(2, "cpu"))):
        toks = [t.float() for t in w.tokens]
        cu = w.cu_seqlens.tolist()
        states = w.state_pool.float()
        wkv7_torch_packed(*toks, cu, states)   # warm-up
        times = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            wkv7_torch_packed(*toks, cu, states)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        legs[name] = {"tokens_per_s": round(w.total_tokens / med, 1),
                      "median_ms": round(med * 1e3, 3), "tokens": w.total_tokens,
                      "repeats": repeats}
    return {"kind": "port", "code": "oracle/torch_loop.py (per-token fp32 loop, heads vectorised)",
            "threads": threads, "legs": legs}


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE measurement (profiles/hbm_traffic.json),
    or None when that kernel/workload pair was not measured."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    k = data["kernels"].get(kernel)
    if k is None or k["workload"] != workload:
        return None
    return int(k["fetch_kib"] * 1024 * data["fetch_scale"] + k["write_kib"] * 1024 * data["write_scale"])


TRAFFIC_SOURCE = ("profiles/hbm_traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of the "
                  "same kernel and workload, scaled by a copy kernel; committed, not measured "
                  "in this run")


def roofline_obj(bytes_per_launch: int, kernel_ms: float, traffic=None):
    achieved = bytes_per_launch / (kernel_ms * 1e-3) / 1e9
    out = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}
    if traffic is not None:
        out["traffic_source"] = TRAFFIC_SOURCE
    return out


def time_fp16_state_decode(torch, flashrwkv2_amd, w, steps: int, warmup: int):
    """Per-step and per-launch times (ms) of the FP16-state recurrence on a
    decode workload: public entry with a reused ticket, then direct C-ABI
    launches between HIP events on the launch stream."""
    from flashrwkv2_amd import _native as N

    state = w.state_pool.half().contiguous()
    state0 = state.clone()
    elapsed = torch.zeros(state.shape[0], dtype=torch.int32, device=state.device)
    out = torch.empty_like(w.v)
    ticket = flashrwkv2_amd.prepare_tmix_wkv7_recurrent_metadata(
        w.cu_seqlens, w.state_indices, total_tokens=w.total_tokens,
        state_pool_size=state.shape[0])
    C = flashrwkv2_amd._C

    def step():
        C.tmix_wkv7_recurrent_fp16_from_decay_logits(
            w.cu_seqlens, w.state_indices, elapsed, state, *w.tokens, out, 1.0, None, ticket)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    state.copy_(state0)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = max(start.elapsed_time(end), (time.perf_counter() - t0) * 1e3) / steps
    lib = N.load()
    stream = torch.cuda.current_stream()
    args = (ticket._query_start_loc_snapshot().data_ptr(), ticket._state_indices_snapshot().data_ptr(),
            ticket._status().data_ptr(), elapsed.data_ptr(), w.state_indices.numel(), w.num_heads,
            64, w.total_tokens, ticket._max_seqlen(), state.data_ptr(),
            *(t.data_ptr() for t in w.tokens[:2]), None, *(t.data_ptr() for t in w.tokens[2:]),
            out.data_ptr(), 1.0, stream.cuda_stream)
    state.copy_(state0)
    torch.cuda.synchronize()
    # the state-streaming kernel alone (the update half of the entry, without
    # the separate elapsed-advance launch)
    start.record(stream)
    for _ in range(steps * 4):
        rc = lib.fr2_wkv7_recurrent_fp16_update(*args)
        if rc:
            N.check(rc, "fr2_wkv7_recurrent_fp16_update")
    end.record(stream)
    torch.cuda.synchronize()
    return ms, start.elapsed_time(end) / (steps * 4)


def time_fp16_state_prefill(torch, flashrwkv2_amd, steps: int):
    """The FP16-state ("Albatross") recurrence on BASELINE config 1's shape
    (8 x 4096 tokens, H = 32, fp16 tokens and an fp16 state pool): the public
    entry (update + elapsed advance) with a reused ticket, and the token-serial
    kernels forced through the C ABI: the barrier-free one (the policy's) and
    the workgroup kernel with a barrier per token.  Per-token fp16 rounding of
    the state makes this contract serial by construction."""
    from flashrwkv2_amd import _native as N
    from flashrwkv2_amd import workloads

    w = workloads.config(1, "cuda", dtype=torch.float16)
    state = w.state_pool.half().contiguous()
    state0 = state.clone()
    elapsed = torch.zeros(state.shape[0], dtype=torch.int32, device=state.device)
    out = torch.empty_like(w.v)
    ticket = flashrwkv2_amd.prepare_tmix_wkv7_recurrent_metadata(
        w.cu_seqlens, w.state_indices, total_tokens=w.total_tokens,
        state_pool_size=state.shape[0])
    C = flashrwkv2_amd._C

    def public():
        C.tmix_wkv7_recurrent_fp16_from_decay_logits(
            w.cu_seqlens, w.state_indices, elapsed, state, *w.tokens, out, 1.0, None, ticket)

    ms = _events_ms(torch, public, steps)
    lib = N.load()
    sh = torch.cuda.current_stream().cuda_stream
    args = (ticket._query_start_loc_snapshot().data_ptr(),
            ticket._state_indices_snapshot().data_ptr(), ticket._status().data_ptr(),
            elapsed.data_ptr(), w.state_indices.numel(), w.num_heads, 64, w.total_tokens,
            ticket._max_seqlen(), state.data_ptr(), *(t.data_ptr() for t in w.tokens[:2]), None,
            *(t.data_ptr() for t in w.tokens[2:]), out.data_ptr(), 1.0, sh)
    forced = {}
    for kern, name in ((6, "serial64h_kernel<IoF16>"),
                       (0, "serial_kernel<64,IoF16,StF16,8>")):
        state.copy_(state0)
        fms = _events_ms(torch, lambda k=kern: N.check(
            lib.fr2_wkv7_recurrent_fp16_update_kernel(k, *args),
            "fr2_wkv7_recurrent_fp16_update_kernel"), max(3, steps // 2), warmup=2)
        forced[name] = fms
    nbytes = (w.total_tokens * w.num_heads * BYTES_PER_TOKEN_HEAD
              + 2 * w.state_indices.numel() * w.num_heads * 64 * 64 * 2)
    kms = forced["serial64h_kernel<IoF16>"]
    out_obj = {
        "workload": w.name + "_fp16_state", "ms_per_step": round(ms, 4),
        "tokens_per_s": round(w.total_tokens / (ms * 1e-3), 1),
        "kernel": "serial64h_kernel<IoF16>", "kernel_ms": round(kms, 4),
        "roofline": roofline_obj(nbytes, kms), "algorithmic_bytes": nbytes,
        "forced_ms": {k: round(v, 4) for k, v in forced.items()},
        "speedup_over_workgroup_kernel": round(forced["serial_kernel<64,IoF16,StF16,8>"] / kms, 3),
    }
    del w, state, state0, out, ticket
    torch.cuda.empty_cache()
    return out_obj


def time_graph_decode(torch, flashrwkv2_amd, w, steps: int = 16, reps: int = 20):
    """Serving-style decode loop on the graph-ticket path: `steps` consecutive
    T=1 steps (device-side metadata validation + recurrence each) captured in
    one HIP graph.  Returns per-step ms for graph replay and for the same
    steps issued eagerly."""
    from flashrwkv2_amd.tmix.wkv7 import (infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
                                          prepare_tmix_wkv7_recurrent_metadata as prep)

    n = w.state_indices.numel()
    dev = w.r.device
    state0 = w.state_pool
    state = state0.clone()
    n_tok = torch.full((1,), w.total_tokens, device=dev, dtype=torch.int32)
    n_seq = torch.full((1,), n, device=dev, dtype=torch.int32)
    live = dict(state_pool_size=state.shape[0], token_capacity=w.total_tokens,
                sequence_capacity=n, max_seqlen_capacity=1, num_active_tokens=n_tok,
                num_active_sequences=n_seq)

    def loop():
        for _ in range(steps):
            t = prep(w.cu_seqlens, w.state_indices, **live)
            wkv7(*w.tokens, state_pool=state, cu_seqlens=w.cu_seqlens,
                 state_indices=w.state_indices, validated_metadata=t)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        loop()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        loop()
    state.copy_(state0)
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    g_ms = max(start.elapsed_time(end), (time.perf_counter() - t0) * 1e3) / (reps * steps)
    t0 = time.perf_counter()
    start.record()
    for _ in range(reps):
        loop()
    end.record()
    torch.cuda.synchronize()
    e_ms = max(start.elapsed_time(end), (time.perf_counter() - t0) * 1e3) / (reps * steps)
    del graph
    return {"workload": w.name + "_graph_loop", "steps_per_graph": steps,
            "graph_ms_per_step": round(g_ms, 5), "eager_ms_per_step": round(e_ms, 5),
            "graph_tokens_per_s": round(w.total_tokens / (g_ms * 1e-3), 1),
            "eager_tokens_per_s": round(w.total_tokens / (e_ms * 1e-3), 1)}


def time_layer_stages(torch, tokens: int, heads: int, steps: int = 20):
    """HBM rates of the fused elementwise stages either side of the
    recurrence on a config-1-sized token block ([tokens, heads*64] fp16):
    kk/a gate (reads k, a12; writes key, a, b: 10 B per element), value
    residual (reads value, v_first, v12; writes value: 8 B) and the readout
    prelinear stage (reads wkv output, r, k, v, gate; writes 1: 12 B).
    Per-launch times from HIP events around direct C-ABI launches."""
    from flashrwkv2_amd import _native as N

    D = 64
    C = heads * D
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(3001)

    def t(*shape):
        return torch.randn(shape, generator=g, device=dev).half()

    lib = N.load()
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    k, a12, v, vf, v12, x, r, gt = (t(tokens, C) for _ in range(8))
    kk, a0, ka, v0, rk, lw, lb = (t(C) for _ in range(7))
    o1, o2, o3 = (torch.empty_like(k) for _ in range(3))
    cases = {
        "kk_a_gate_kernel<64>": (
            10, lambda: lib.fr2_tmix_kk_a_gate_forward(
                tokens, heads, D, k.data_ptr(), kk.data_ptr(), a0.data_ptr(), a12.data_ptr(),
                ka.data_ptr(), o1.data_ptr(), o2.data_ptr(), o3.data_ptr(), sh)),
        "vres_kernel": (
            8, lambda: lib.fr2_tmix_vres_forward(tokens, C, v.data_ptr(), vf.data_ptr(),
                                                 v0.data_ptr(), v12.data_ptr(), o1.data_ptr(), sh)),
        "readout_prelinear_kernel<64>": (
            12, lambda: lib.fr2_tmix_readout_prelinear_forward(
                tokens, heads, D, x.data_ptr(), r.data_ptr(), k.data_ptr(), v.data_ptr(),
                rk.data_ptr(), lw.data_ptr(), lb.data_ptr(), gt.data_ptr(), o2.data_ptr(), sh)),
    }
    out = {}
    for name, (bpe, fn) in cases.items():
        N.check(fn(), name)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        nbytes = bpe * tokens * C
        wl = f"cfg1_tokens{tokens}_C{C}_fp16"
        out[name] = {"kernel_ms": round(ms, 5), "algorithmic_bytes": nbytes,
                     "roofline": roofline_obj(nbytes, ms, measured_traffic(name, wl))}
    return {"workload": f"cfg1_tokens{tokens}_C{C}_fp16", "kernels": out}


def time_kk_fused(torch, flashrwkv2_amd, steps: int, serving: bool = False):
    """wkv_prepare's kk / a-gate stage and the recurrence in fp16 on BASELINE
    config 1's shape (8 x 4096 tokens, H = 32; the workgroup-per-unit
    chunked kernel) or, with `serving`, on a serving batch of 2 048
    sequences x 100 tokens (65 536 units; the wavefront-per-unit kernel): the
    reference's two kernels (kk_a_gate_kernel writes key, a, b; the
    recurrence reads them back) against the chunked kernel that forms them in
    its load stage.  Both read the projected key and a12 and write the gated
    key and y, so the fused form moves 14 B per (token, channel) where the
    pair moves 24 B.  With the readout's elementwise stage (GroupNorm, the
    r k' r_k residual, the gate) also in the kernel's write-back: three
    kernels move 36 B per (token, channel), the fused one 16 B (it reads the
    gate and writes the readout instead of y)."""
    from flashrwkv2_amd import _C as CC
    from flashrwkv2_amd import _native as N
    from flashrwkv2_amd import workloads

    if serving:
        n_seq, length, heads = 2048, 100, 32
        toks = workloads.make_tokens(n_seq * length, heads, u_range=(-6.0, -0.5), seed=3003,
                                     device="cuda", dtype=torch.float16)
        w = workloads._pack(f"serving_S{n_seq}_T{length}_H{heads}_fp16_kk_gate", toks,
                            [length] * n_seq, heads, 0.1, 3003, "cuda", {})
        rec_kernel, kk_kernel, ro_kernel = (
            "chunk64w_kernel<IoF16,false>", "chunk64w_kernel<IoF16,false,false,true>",
            "chunk64w_kernel<IoF16,false,false,true,true>")
        name = w.name
    else:
        w = workloads.config(1, "cuda", dtype=torch.float16)
        rec_kernel, kk_kernel, ro_kernel = (
            "chunk64r_kernel<IoF16>", "chunk64r_kernel<IoF16,kk>",
            "chunk64_kernel<IoF16,false,false,false,true,true>")
        name = "cfg1_prefill_B8_T4096_H32_fp16_kk_gate"
    T, H, D = w.total_tokens, w.num_heads, 64
    C = H * D
    g = torch.Generator(device="cuda")
    g.manual_seed(3002)
    r, logits, _, v, _, _ = w.tokens
    k = (torch.randn((T, H, D), generator=g, device="cuda") * 0.7).half()
    a12 = torch.randn((T, H, D), generator=g, device="cuda").half()
    kk = (torch.randn(C, generator=g, device="cuda") * 0.2 + 0.85).half()
    a0 = (torch.randn(C, generator=g, device="cuda") * 0.5).half()
    ka = torch.rand(C, generator=g, device="cuda").half()
    state = w.state_pool.clone()
    new_k, a, b, out = (torch.empty_like(k) for _ in range(4))
    ticket = flashrwkv2_amd.prepare_tmix_wkv7_recurrent_metadata(
        w.cu_seqlens, w.state_indices, total_tokens=T, state_pool_size=state.shape[0])
    lib = N.load()
    sh = torch.cuda.current_stream().cuda_stream

    def two_stage():
        N.check(lib.fr2_tmix_kk_a_gate_forward(
            T, H, D, k.data_ptr(), kk.data_ptr(), a0.data_ptr(), a12.data_ptr(), ka.data_ptr(),
            new_k.data_ptr(), a.data_ptr(), b.data_ptr(), sh), "fr2_tmix_kk_a_gate_forward")
        CC.tmix_wkv7_recurrent_fp32_from_decay_logits(
            w.cu_seqlens, w.state_indices, state, r, logits, new_k, v, a, b, out, 1.0, None,
            ticket)

    def fused():
        CC.tmix_wkv7_recurrent_fp32_from_kk_gate(
            w.cu_seqlens, w.state_indices, state, r, logits, k, v, a12, kk, a0, ka, new_k, out,
            1.0, None, ticket)

    seqs = w.state_indices.numel()
    state_bytes = 2 * seqs * H * D * D * 4
    fused_bytes = 14 * T * C + state_bytes
    pair_bytes = 24 * T * C + state_bytes
    def recurrence():
        CC.tmix_wkv7_recurrent_fp32_from_decay_logits(
            w.cu_seqlens, w.state_indices, state, r, logits, new_k, v, a, b, out, 1.0, None,
            ticket)

    gate = torch.sigmoid(torch.randn((T, H, D), generator=g, device="cuda")).half()
    rk = (torch.randn(C, generator=g, device="cuda") * 0.3).half()
    lnw = (1.0 + 0.1 * torch.randn(C, generator=g, device="cuda")).half()
    lnb = (0.1 * torch.randn(C, generator=g, device="cuda")).half()
    ro = torch.empty_like(k)

    def three_stage():
        two_stage()
        N.check(lib.fr2_tmix_readout_prelinear_forward(
            T, H, D, out.data_ptr(), r.data_ptr(), new_k.data_ptr(), v.data_ptr(), rk.data_ptr(),
            lnw.data_ptr(), lnb.data_ptr(), gate.data_ptr(), ro.data_ptr(), sh),
            "fr2_tmix_readout_prelinear_forward")

    def fused_ro():
        CC.tmix_wkv7_recurrent_fp32_from_kk_gate_readout(
            w.cu_seqlens, w.state_indices, state, r, logits, k, v, a12, gate, kk, a0, ka, rk,
            lnw, lnb, new_k, ro, None, 1.0, None, ticket)

    two_ms = _events_ms(torch, two_stage, steps)
    fused_ms = _events_ms(torch, fused, steps)
    rec_ms = _events_ms(torch, recurrence, steps)
    three_ms = _events_ms(torch, three_stage, steps)
    fused_ro_ms = _events_ms(torch, fused_ro, steps)
    three_bytes = 36 * T * C + state_bytes
    fused_ro_bytes = 16 * T * C + state_bytes
    out_obj = {
        "workload": name, "total_tokens": T,
        "two_stage": {"ms_per_step": round(two_ms, 4),
                      "kernels": f"kk_a_gate_kernel<64> + {rec_kernel}",
                      "algorithmic_bytes": pair_bytes,
                      "roofline": roofline_obj(pair_bytes, two_ms)},
        "fused": {"ms_per_step": round(fused_ms, 4),
                  "kernel": kk_kernel,
                  "algorithmic_bytes": fused_bytes,
                  "roofline": roofline_obj(fused_bytes, fused_ms)},
        "recurrence_alone_ms": round(rec_ms, 4),
        "saved_ms": round(two_ms - fused_ms, 4),
        "with_readout": {
            "three_stage": {"ms_per_step": round(three_ms, 4),
                            "kernels": f"kk_a_gate_kernel<64> + {rec_kernel} + "
                                       "readout_prelinear_kernel<64>",
                            "algorithmic_bytes": three_bytes,
                            "roofline": roofline_obj(three_bytes, three_ms)},
            "fused": {"ms_per_step": round(fused_ro_ms, 4),
                      "kernel": ro_kernel,
                      "algorithmic_bytes": fused_ro_bytes,
                      "roofline": roofline_obj(fused_ro_bytes, fused_ro_ms)},
            "saved_ms": round(three_ms - fused_ro_ms, 4),
        },
    }
    del w, state, k, a12, new_k, a, b, out, ticket, gate, ro
    torch.cuda.empty_cache()
    return out_obj


# Algorithmic HBM bytes of the training backward per (token, head) at D=64:
# reads r, w, k, v, a, b, dy (7 x 2D bf16), sa (4D fp32) and the forward's
# boundary snapshot amortised over its 16 tokens (4 D^2 / 16); writes the six
# bf16 gradients (6 x 2D).
BWD_BYTES_PER_TOKEN_HEAD = 7 * 128 + 256 + 64 * 64 * 4 // 16 + 6 * 128


def time_long_context(torch, flashrwkv2_amd, steps: int):
    """BASELINE config 4 at full size (B=1, T=65536, H=64): the public call,
    which cuts the sequence into pieces (summary pass, combine, pieces), and
    the unsplit chunked kernel (one block per head) through the C ABI."""
    from flashrwkv2_amd import _C as CC
    from flashrwkv2_amd import workloads

    w = workloads.config(4, "cuda")
    run = Runner(w, torch, flashrwkv2_amd)
    ms = run.time_steps(steps, 2)
    unsplit_ms = run.time_kernel(max(2, steps // 2))
    pieces, piece_len, lead_len, ws = CC.split_plan(w.state_indices.numel(), w.num_heads, 64,
                                                    run.ticket._max_seqlen())
    nbytes = algorithmic_bytes(w.total_tokens, w.num_heads, w.state_indices.numel())
    out = {
        "workload": w.name, "ms_per_step": round(ms, 4),
        "tokens_per_s": round(w.total_tokens / (ms * 1e-3), 1),
        "kernels": "chunk64r_kernel piece 0 (second stream) concurrent with the summary pass "
                   "(chunk64_kernel), split_combine_kernel, chunk64r_kernel pieces 1..P-1",
        "pieces": pieces, "piece_len": piece_len, "lead_len": lead_len, "workspace_bytes": ws,
        "roofline": roofline_obj(nbytes, ms, measured_traffic(
            "split:lead+summary+combine+pieces", w.name)),
        "unsplit": {"ms_per_step": round(unsplit_ms, 4),
                    "tokens_per_s": round(w.total_tokens / (unsplit_ms * 1e-3), 1),
                    "kernel": "chunk64r_kernel<IoBF16> (one block per head)",
                    "roofline": roofline_obj(nbytes, unsplit_ms)},
        "algorithmic_bytes": nbytes,
    }
    del run, w
    torch.cuda.empty_cache()
    return out


def time_varlen(torch, flashrwkv2_amd, steps: int):
    """BASELINE config 3 (64 packed sequences of seeded lengths U{1..2048},
    H = 64, per-sequence fp32 states): the public call with a reused ticket,
    and the kernel's per-launch time through the C ABI."""
    from flashrwkv2_amd import workloads

    w = workloads.config(3, "cuda")
    run = Runner(w, torch, flashrwkv2_amd)
    ms = run.time_steps(steps, 5)
    kms = run.time_kernel(steps)
    nbytes = algorithmic_bytes(w.total_tokens, w.num_heads, w.state_indices.numel())
    out = {
        "workload": w.name, "total_tokens": w.total_tokens,
        "ms_per_step": round(ms, 4), "tokens_per_s": round(w.total_tokens / (ms * 1e-3), 1),
        "kernel_ms": round(kms, 4), "kernel": run.kernel_name(),
        "roofline": roofline_obj(nbytes, kms), "algorithmic_bytes": nbytes,
    }
    del run, w
    torch.cuda.empty_cache()
    return out


def time_mid_length(torch, flashrwkv2_amd, steps: int, n: int = 2048, length: int = 100,
                    heads: int = 32):
    """Serving-style batch of many mid-length sequences (2048 x 100 tokens,
    H = 32, per-sequence fp32 states ~ N(0, 0.1)): the public call (which the
    library dispatches by max_seqlen and unit count) and the candidate
    kernels forced, the measurements behind the policy."""
    from flashrwkv2_amd import workloads

    toks = workloads.make_tokens(n * length, heads, u_range=(-6.0, -0.5), seed=1005,
                                 device="cuda")
    w = workloads._pack(f"mid_S{n}_T{length}_H{heads}", toks, [length] * n, heads, 0.1, 1005,
                        "cuda", {"S": n, "T": length, "H": heads})
    run = Runner(w, torch, flashrwkv2_amd)
    ms = run.time_steps(steps, 5)
    kms = run.time_kernel(steps)
    nbytes = algorithmic_bytes(w.total_tokens, w.num_heads, w.state_indices.numel())
    forced = {}
    for kern, name in ((0, "serial64w_kernel<IoBF16,StF32>"), (2, "chunk64r_kernel<IoBF16>"),
                       (4, "chunk64w_kernel<IoBF16,false>")):
        f = lambda k=kern: run.C.tmix_wkv7_recurrent_fp32_kernel_forced(
            k, w.cu_seqlens, w.state_indices, run.state, *w.tokens, run.out, 1.0, None,
            run.ticket)
        fms = _events_ms(torch, f, steps)
        forced[name] = {"kernel_ms": round(fms, 4), "roofline": roofline_obj(nbytes, fms)}
    out = {
        "workload": w.name, "total_tokens": w.total_tokens,
        "ms_per_step": round(ms, 4), "tokens_per_s": round(w.total_tokens / (ms * 1e-3), 1),
        "kernel_ms": round(kms, 4), "kernel": run.kernel_name(),
        "roofline": roofline_obj(nbytes, kms, measured_traffic(run.kernel_name(), w.name)),
        "algorithmic_bytes": nbytes,
        "forced": forced,
    }
    del run, w, toks
    torch.cuda.empty_cache()
    return out


def time_short_batches(torch, flashrwkv2_amd, steps: int, heads: int = 32):
    """Short-sequence batches at both ends of the dispatch policy
    (csrc/api.hip run_family), each through the public call and with every
    kernel family forced: many 16-token sequences (65 536 (sequence, head)
    units: the chunked kernel with one wave per unit) and 8 sequences of 16
    tokens (256 units: the chunked kernel with one workgroup per unit)."""
    from flashrwkv2_amd import workloads

    out = []
    for n, length in ((2048, 16), (8, 16)):
        toks = workloads.make_tokens(n * length, heads, u_range=(-6.0, -0.5), seed=1006,
                                     device="cuda")
        w = workloads._pack(f"short_S{n}_T{length}_H{heads}", toks, [length] * n, heads, 0.1,
                            1006, "cuda", {"S": n, "T": length, "H": heads})
        run = Runner(w, torch, flashrwkv2_amd)
        ms = run.time_steps(steps, 5)
        nbytes = algorithmic_bytes(w.total_tokens, w.num_heads, w.state_indices.numel())
        forced = {}
        for kern, name in ((0, "serial64w_kernel<IoBF16,StF32>"),
                           (1, "decode64_kernel<IoBF16,StF32>"),
                           (2, "chunk64r_kernel<IoBF16>"),
                           (4, "chunk64w_kernel<IoBF16,false>")):
            f = lambda k=kern: run.C.tmix_wkv7_recurrent_fp32_kernel_forced(
                k, w.cu_seqlens, w.state_indices, run.state, *w.tokens, run.out, 1.0, None,
                run.ticket)
            fms = _events_ms(torch, f, steps)
            forced[name] = {"kernel_ms": round(fms, 5), "roofline": roofline_obj(nbytes, fms)}
        out.append({"workload": w.name, "units": n * heads, "ms_per_step": round(ms, 5),
                    "kernel": run.kernel_name(), "roofline": roofline_obj(nbytes, ms),
                    "algorithmic_bytes": nbytes, "forced": forced})
        del run, w, toks
    torch.cuda.empty_cache()
    return out


def _events_ms(torch, fn, launches: int, warmup: int = 5) -> float:
    """Average duration (ms) of `fn` over `launches` back-to-back calls on the
    current stream, HIP events on both sides (and the wall clock, whichever
    is longer)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(launches):
        fn()
    end.record()
    torch.cuda.synchronize()
    return max(start.elapsed_time(end), (time.perf_counter() - t0) * 1e3) / launches


VALU_FP32_PEAK_TFLOPS = 157.3      # vendor figure (packed fp32)
FLOPS_PER_TOKEN_HEAD = 5 * 64 * 64 * 2   # recurrence form: 5 x D x D FMA


def time_other_paths(torch, flashrwkv2_amd, w, steps: int):
    """The remaining forward paths on the config-1 batch, through the C ABI
    on the current stream: the token-serial kernel forced (what D = 128/256
    and mid-length sequences run), and the rl_infctx forward (chunk list of
    16-token chunks, one block per sequence) and its backward replay (every
    chunk from its start-of-chunk state, sa written)."""
    from flashrwkv2_amd import _native as N
    from flashrwkv2_amd.tmix.wkv7.rl_infctx import _chunk_table

    lib = N.load()
    stream = torch.cuda.current_stream().cuda_stream
    B, H, T = w.state_indices.numel(), w.num_heads, w.total_tokens
    toks = [t.data_ptr() for t in w.tokens]
    out = torch.empty_like(w.v)
    ticket = flashrwkv2_amd.prepare_tmix_wkv7_recurrent_metadata(
        w.cu_seqlens, w.state_indices, total_tokens=T, state_pool_size=B)
    state = torch.zeros((B, H, 64, 64), device="cuda", dtype=torch.float32)
    meta = (ticket._query_start_loc_snapshot().data_ptr(),
            ticket._state_indices_snapshot().data_ptr(), ticket._status().data_ptr())

    def serial():
        N.check(lib.fr2_wkv7_recurrent_fp32_forward_kernel(
            N.KERNEL_SERIAL, *meta, B, H, 64, T, ticket._max_seqlen(), N.FR2_DTYPE_BFLOAT16,
            state.data_ptr(), toks[0], toks[1], None, *toks[2:], out.data_ptr(), 1.0, stream),
            "serial")

    offsets = w.cu_seqlens.cpu().tolist()
    seq_chunks, starts, ends = _chunk_table(w.cu_seqlens.cpu().to(torch.int64), 16, w.r.device)
    nchunks = starts.numel()

    def rl_forward():
        N.check(lib.fr2_wkv7_rl_infctx_forward(
            seq_chunks.data_ptr(), starts.data_ptr(), ends.data_ptr(), B, nchunks, H, 64, T,
            max(hi - lo for lo, hi in zip(offsets[:-1], offsets[1:])), 16, 1,
            N.FR2_DTYPE_BFLOAT16, state.data_ptr(), toks[0], toks[1], None, *toks[2:],
            out.data_ptr(), 1.0, stream), "rl_infctx forward")

    g = torch.Generator(device="cuda").manual_seed(5)
    boundary = torch.randn((nchunks, H, 64, 64), device="cuda", generator=g) * 0.1
    sa = torch.empty((T, H, 64), device="cuda", dtype=torch.float32)

    def rl_replay():
        N.check(lib.fr2_wkv7_rl_infctx_replay(
            starts.data_ptr(), ends.data_ptr(), nchunks, H, 64, T, N.FR2_DTYPE_BFLOAT16,
            boundary.data_ptr(), toks[0], toks[1], None, *toks[2:], out.data_ptr(),
            sa.data_ptr(), 1.0, stream), "rl_infctx replay")

    n = max(5, steps // 2)
    s_ms = _events_ms(torch, serial, n)
    f_ms = _events_ms(torch, rl_forward, n)
    r_ms = _events_ms(torch, rl_replay, n)
    io = T * H * BYTES_PER_TOKEN_HEAD
    flops = T * H * FLOPS_PER_TOKEN_HEAD
    replay_bytes = io + T * H * 64 * 4 + nchunks * H * STATE_BYTES   # + sa, + boundary reads
    out_obj = {
        "workload": w.name,
        "token_serial": {
            "kernel": "serial64w_kernel<IoBF16,StF32>", "kernel_ms": round(s_ms, 4),
            "tokens_per_s": round(T / (s_ms * 1e-3), 1),
            "roofline": roofline_obj(io + 2 * B * H * STATE_BYTES, s_ms),
            "valu": {"achieved_tflops": round(flops / (s_ms * 1e-3) / 1e12, 2),
                     "peak_tflops": VALU_FP32_PEAK_TFLOPS,
                     "frac": round(flops / (s_ms * 1e-3) / 1e12 / VALU_FP32_PEAK_TFLOPS, 4),
                     "flops_per_token_head": FLOPS_PER_TOKEN_HEAD},
        },
        "rl_infctx_forward": {
            "kernel": "chunk64_kernel<IoBF16,false> over each sequence's chunk list",
            "chunk_size": 16, "kernel_ms": round(f_ms, 4),
            "tokens_per_s": round(T / (f_ms * 1e-3), 1),
            "roofline": roofline_obj(io + 2 * B * H * STATE_BYTES, f_ms),
        },
        "rl_infctx_replay": {
            "kernel": "chunk64w_kernel<IoBF16,false,true>: one wavefront per (16-token chunk, head), sa written",
            "chunks": nchunks, "kernel_ms": round(r_ms, 4),
            "tokens_per_s": round(T / (r_ms * 1e-3), 1),
            "roofline": roofline_obj(replay_bytes, r_ms), "algorithmic_bytes": replay_bytes,
        },
    }
    del boundary, sa, out, state
    torch.cuda.empty_cache()
    return out_obj


def time_chunk_bf16_state(torch, flashrwkv2_amd, w, steps: int):
    """The bf16-state chunk entry (infer_tmix_wkv7_chunk_bf16_forward_varlen)
    on a config-1-shaped batch with a bf16 state pool: public calls with a
    reused ticket between HIP events."""
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_chunk_bf16_forward_varlen as fn

    pool = w.state_pool.to(torch.bfloat16) if w.state_pool is not None else torch.zeros(
        (w.state_indices.numel(), w.num_heads, 64, 64), device=w.r.device, dtype=torch.bfloat16)
    ticket = flashrwkv2_amd.prepare_tmix_wkv7_recurrent_metadata(
        w.cu_seqlens, w.state_indices, total_tokens=w.total_tokens, state_pool_size=pool.shape[0])

    def call():
        return fn(*w.tokens, state_pool=pool, cu_seqlens=w.cu_seqlens,
                  state_indices=w.state_indices, validated_metadata=ticket)

    # warm-up as long as the prefill leg's (~70 ms): after the short decode
    # legs the clocks need that long to come back up
    for _ in range(200):
        call()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        call()
    end.record()
    torch.cuda.synchronize()
    ms = max(start.elapsed_time(end), (time.perf_counter() - t0) * 1e3) / steps
    nbytes = (w.total_tokens * w.num_heads * BYTES_PER_TOKEN_HEAD
              + 2 * w.state_indices.numel() * w.num_heads * STATE_BYTES // 2)   # bf16 state
    return {"workload": w.name + "_bf16_state", "ms_per_step": round(ms, 5),
            "tokens_per_s": round(w.total_tokens / (ms * 1e-3), 1),
            "kernel": "chunk64_kernel<IoBF16,false> (bf16 state load/store)",
            "roofline": roofline_obj(nbytes, ms)}


def _bwd_traffic(B, T, H):
    """Measured HBM bytes of the two backward kernels (PMC, committed), when
    the workload is the measured one."""
    wl = f"cfg1_shape_training_B{B}_T{T}_H{H}"
    parts = [measured_traffic(k, wl) for k in ("chunk64r_kernel<IoBF16,false,true>", "key_chunk_kernel")]
    return None if any(x is None for x in parts) else sum(parts)


def _launch_ms(torch, stream, call, name, steps, warmup=5, passes=3):
    """Per-launch time (ms) of a C-ABI call returning a status: `warmup`
    untimed launches, then `passes` passes of `steps` launches, each between
    HIP events on the launch stream; the median pass."""
    from flashrwkv2_amd import _native as N

    for _ in range(warmup):
        N.check(call(), name)
    torch.cuda.synchronize()
    per = []
    for _ in range(passes):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            rc = call()
            if rc:
                N.check(rc, name)
        end.record(stream)
        torch.cuda.synchronize()
        per.append(start.elapsed_time(end) / steps)
    return sorted(per)[len(per) // 2]


def lib_ws(B, T, H, D):
    from flashrwkv2_amd import _native as N

    return int(N.load().fr2_wkv7_pretrain_backward_workspace_floats(B, T, H, D))


def time_pretrain_training(torch, w, steps: int):
    """The [B,T,H,D] training path on a config-1-shaped batch: per-launch
    times (ms) of the forward (y, state_dot_a, boundary) and of the backward
    (two kernels) through the C ABI: the median of three passes of `steps`
    launches between HIP events on the launch stream, after five warm-up
    launches (`_launch_ms`)."""
    from flashrwkv2_amd import _native as N

    B, T, H = w.info["B"], w.info["T"], w.info["H"]
    D = 64
    toks = [t.view(B, T, H, D) for t in w.tokens]
    g = torch.Generator(device=toks[0].device)
    g.manual_seed(2001)
    dy = torch.randn((B, T, H, D), generator=g, device=toks[0].device).to(torch.bfloat16)
    y = torch.empty_like(toks[3])
    boundary = torch.empty((B, H, T // 16, D, D), device=y.device, dtype=torch.float32)
    sa = torch.empty((B, T, H, D), device=y.device, dtype=torch.float32)
    work = torch.empty(lib_ws(B, T, H, D), device=y.device, dtype=torch.float32)
    grads = [torch.empty_like(t) for t in toks]
    lib = N.load()
    stream = torch.cuda.current_stream()
    ptrs = [t.data_ptr() for t in toks]
    fwd_args = (B, T, H, D, *ptrs, y.data_ptr(), boundary.data_ptr(), sa.data_ptr(),
                stream.cuda_stream)
    bwd_args = (B, T, H, D, *ptrs, dy.data_ptr(), boundary.data_ptr(), sa.data_ptr(),
                work.data_ptr(), *(t.data_ptr() for t in grads), stream.cuda_stream)

    def timed(fn, args, name):
        return _launch_ms(torch, stream, lambda: fn(*args), name, steps)

    fwd_ms = timed(lib.fr2_wkv7_pretrain_forward, fwd_args, "fr2_wkv7_pretrain_forward")
    bwd_ms = timed(lib.fr2_wkv7_pretrain_backward, bwd_args, "fr2_wkv7_pretrain_backward")
    ok = all(bool(torch.isfinite(t).all()) for t in grads)
    bwd_bytes = BWD_BYTES_PER_TOKEN_HEAD * B * T * H
    return {
        "workload": f"cfg1_shape_training_B{B}_T{T}_H{H}",
        "forward_ms": round(fwd_ms, 4), "backward_ms": round(bwd_ms, 4),
        "train_tokens_per_s": round(B * T / ((fwd_ms + bwd_ms) * 1e-3), 1),
        "backward_tokens_per_s": round(B * T / (bwd_ms * 1e-3), 1),
        "backward_algorithmic_bytes": bwd_bytes,
        "backward_roofline": roofline_obj(bwd_bytes, bwd_ms, _bwd_traffic(B, T, H)),
        "gradients_finite": ok,
        "kernels": ["chunk64_kernel<IoBF16,true> (forward: y, sa, boundary)",
                    "chunk64r_kernel<IoBF16,false,true> (value pass: dv, dsa, P snapshots)",
                    "key_chunk_kernel (key pass: dr, dw, dk, db, da)"],
    }


# StateTune HBM bytes per (token, head) at D = 64 with 16-bit tokens:
#   forward  r w k a b v in (6 x 128 B), y out (128 B), state_dot_a out (256 B)
#   backward replay: r w k a b v in (768 B); value pass: r w k a b dy in
#            (768 B), dv (128 B) + dsa (256 B) out; key pass: dy v (256 B),
#            sa dsa (512 B), r w k a b (640 B) in, five gradients (640 B) out
# plus, per chunk and head, the 16 KiB boundary (written forward, read twice
# backward) and, per 16 tokens and head, the 16 KiB replay snapshot (written
# and read once).
ST_FWD_BYTES_PER_TOKEN_HEAD = 6 * 128 + 128 + 256
ST_BWD_BYTES_PER_TOKEN_HEAD = 768 + 768 + 128 + 256 + 256 + 512 + 640 + 640


def time_statetune_ragged(torch, w, steps: int):
    """StateTune on the config-1 shape (8 x 4096 tokens, H = 32) over a
    ragged chunk list: chunks of seeded random lengths 1..700 (most not a
    multiple of 16), a few empty, and 40 tokens of each sequence in no chunk.
    Through the public `_C` entries (the forward builds the padded grid on
    the host from the chunk metadata, then runs the chunked MFMA kernels;
    the backward reuses the grid), per call, HIP events and wall clock; the
    token-serial kernels on the same list for comparison."""
    import numpy as np

    import flashrwkv2_amd._C as CC

    B, T, H = w.info["B"], w.info["T"], w.info["H"]
    D = 64
    dev = w.tokens[0].device
    toks = list(w.tokens)
    rng = np.random.default_rng(2003)
    offsets, starts, ends = [0], [], []
    for b in range(B):
        t, end = b * T, (b + 1) * T - 40
        while t < end:
            n = min(int(rng.integers(0, 701)), end - t)
            starts.append(t)
            ends.append(t + n)
            t += n
        offsets.append(len(starts))
    meta = [torch.tensor(x, dtype=torch.int32, device=dev) for x in (offsets, starts, ends)]
    C = len(starts)
    g = torch.Generator(device=dev)
    g.manual_seed(2004)
    state0 = torch.randn((B, H, D, D), generator=g, device=dev) * 0.1
    state = state0.clone()
    dy = torch.randn((B * T, H, D), generator=g, device=dev).to(torch.bfloat16)
    dfin = torch.randn((B, H, D, D), generator=g, device=dev)
    y = torch.empty_like(toks[3])
    boundary = torch.empty((C, H, D, D), device=dev, dtype=torch.float32)
    sa = torch.empty((B * T, H, D), device=dev, dtype=torch.float32)
    grads = [torch.empty_like(t) for t in toks]
    g0 = torch.empty_like(state)
    res = {}

    def fwd():
        state.copy_(state0)
        res["snap"] = CC.statetune_tmix_wkv7_recurrent_fp32io16_forward(
            *meta, state, *toks, y, boundary, sa, 1.0)

    def bwd():
        CC.statetune_tmix_wkv7_recurrent_fp32io16_backward(
            *meta, state, *toks, sa, dy, dfin, boundary, *grads, g0, 1.0,
            snapshots=res["snap"])

    out = {"workload": f"cfg1_shape_statetune_ragged_B{B}_T{T}_H{H}", "chunks": C,
           "tokens_in_chunks": int(sum(e - s for s, e in zip(starts, ends)))}
    for name, serial in (("chunked", False), ("token_serial", True)):
        CC._statetune_force_serial = serial
        try:
            n = steps if not serial else max(2, steps // 3)
            f_ms = _events_ms(torch, fwd, n, warmup=2)
            b_ms = _events_ms(torch, bwd, n, warmup=2)
        finally:
            CC._statetune_force_serial = False
        out[name] = {"forward_ms": round(f_ms, 4), "backward_ms": round(b_ms, 4),
                     # the chunked forward returns its padded-grid plan for the
                     # backward; the token-serial one returns nothing
                     "path": "padded_chunked" if res["snap"] is not None else "token_serial"}
    out["gradients_finite"] = all(bool(torch.isfinite(t).all()) for t in (*grads, g0))
    del state, dy, y, boundary, sa, grads, res
    torch.cuda.empty_cache()
    return out


def time_statetune_training(torch, w, steps: int, chunk_len: int = 1024):
    """StateTune on the config-1 shape: B sequences of T tokens, each run as
    T/chunk_len chunks from a trainable fp32 initial state ~ N(0, 0.1);
    per-call times (ms) of the forward and of the backward through the C ABI
    between HIP events on the launch stream.  This chunk list is the uniform
    layout, so the public entry runs the chunked MFMA kernels
    (`fr2_wkv7_statetune_uniform_*`); the token-serial kernels that serve
    every other chunk list (`fr2_wkv7_statetune_*`) are timed on it too."""
    from flashrwkv2_amd import _native as N

    B, T, H = w.info["B"], w.info["T"], w.info["H"]
    D = 64
    dev = w.tokens[0].device
    toks = list(w.tokens)
    nck = T // chunk_len
    offsets = torch.arange(B + 1, dtype=torch.int32, device=dev) * nck
    starts = torch.arange(B * nck, dtype=torch.int32, device=dev) * chunk_len
    ends = starts + chunk_len
    C = B * nck
    g = torch.Generator(device=dev)
    g.manual_seed(2002)
    state0 = torch.randn((B, H, D, D), generator=g, device=dev) * 0.1
    state = state0.clone()
    dy = torch.randn((B * T, H, D), generator=g, device=dev).to(torch.bfloat16)
    dfin = torch.randn((B, H, D, D), generator=g, device=dev)
    y = torch.empty_like(toks[3])
    boundary = torch.empty((C, H, D, D), device=dev, dtype=torch.float32)
    sa = torch.empty((B * T, H, D), device=dev, dtype=torch.float32)
    snaps = torch.empty((B, H, T // 16, D, D), device=dev, dtype=torch.float32)
    lib = N.load()
    work_s = torch.empty(int(lib.fr2_wkv7_statetune_backward_workspace_floats(B * T, H, D)),
                         device=dev, dtype=torch.float32)
    work_u = torch.empty(int(lib.fr2_wkv7_statetune_uniform_backward_workspace_floats(B, T, H)),
                         device=dev, dtype=torch.float32)
    grads = [torch.empty_like(t) for t in toks]
    g0 = torch.empty_like(state)
    stream = torch.cuda.current_stream()
    hs = stream.cuda_stream
    meta = (offsets.data_ptr(), starts.data_ptr(), ends.data_ptr(), B, C, B * T, H, D,
            N.FR2_DTYPE_BFLOAT16)
    ptrs = [t.data_ptr() for t in toks]
    gptrs = [t.data_ptr() for t in grads]

    # each forward first restores the initial state (it is updated in place):
    # an 8 MiB copy, about 2 us, inside the forward's timing
    def fwd_uniform():
        state.copy_(state0)
        return lib.fr2_wkv7_statetune_uniform_forward(
            B, T, H, chunk_len, state.data_ptr(), *ptrs, y.data_ptr(), boundary.data_ptr(),
            sa.data_ptr(), snaps.data_ptr(), 1.0, hs)

    def bwd_uniform():
        return lib.fr2_wkv7_statetune_uniform_backward(
            B, T, H, chunk_len, *ptrs, sa.data_ptr(), dy.data_ptr(), dfin.data_ptr(),
            boundary.data_ptr(), snaps.data_ptr(), work_u.data_ptr(), *gptrs, g0.data_ptr(), 1.0,
            hs)

    def fwd_serial():
        state.copy_(state0)
        return lib.fr2_wkv7_statetune_forward(*meta, state.data_ptr(), *ptrs, y.data_ptr(),
                                              boundary.data_ptr(), sa.data_ptr(), 1.0, hs)

    def bwd_serial():
        return lib.fr2_wkv7_statetune_backward(
            *meta, *ptrs, sa.data_ptr(), dy.data_ptr(), dfin.data_ptr(), boundary.data_ptr(),
            work_s.data_ptr(), *gptrs, g0.data_ptr(), 1.0, hs)

    def timed(fn, name):
        return _launch_ms(torch, stream, fn, name, steps)

    sf = timed(fwd_serial, "fr2_wkv7_statetune_forward")
    sb = timed(bwd_serial, "fr2_wkv7_statetune_backward")
    uf = timed(fwd_uniform, "fr2_wkv7_statetune_uniform_forward")
    ub = timed(bwd_uniform, "fr2_wkv7_statetune_uniform_backward")
    ok = all(bool(torch.isfinite(t).all()) for t in (*grads, g0))
    th = B * T * H
    state_bytes = D * D * 4
    # token-serial: boundaries written forward and read by replay and key
    # pass; replay snapshots written and read once
    fwd_bytes = ST_FWD_BYTES_PER_TOKEN_HEAD * th + (C + 2 * B) * H * state_bytes
    bwd_bytes = (ST_BWD_BYTES_PER_TOKEN_HEAD * th + 3 * C * H * state_bytes
                 + 2 * (th // 16) * state_bytes + 2 * B * H * state_bytes)
    # chunked: the forward also writes the post-16-token snapshots, which the
    # backward's key pass reads; the backward is the pretrain one's 2 944 B
    # per token-head plus dL/dS_final in and dL/dS_initial out
    ufwd_bytes = fwd_bytes + (th // 16) * state_bytes
    ubwd_bytes = BWD_BYTES_PER_TOKEN_HEAD * th + 2 * B * H * state_bytes
    return {
        "workload": f"cfg1_shape_statetune_B{B}_T{T}_H{H}_chunk{chunk_len}",
        "forward_ms": round(uf, 4), "backward_ms": round(ub, 4),
        "train_tokens_per_s": round(B * T / ((uf + ub) * 1e-3), 1),
        "forward_roofline": roofline_obj(ufwd_bytes, uf),
        "backward_roofline": roofline_obj(ubwd_bytes, ub),
        "token_serial": {"forward_ms": round(sf, 4), "backward_ms": round(sb, 4),
                         "train_tokens_per_s": round(B * T / ((sf + sb) * 1e-3), 1),
                         "forward_roofline": roofline_obj(fwd_bytes, sf),
                         "backward_roofline": roofline_obj(bwd_bytes, sb)},
        "gradients_finite": ok,
        "kernels": ["chunk64_kernel<IoBF16,true> (forward) + st_gather_kernel (boundaries)",
                    "chunk64r_kernel<IoBF16,false,true> + first_token_kernel + key_chunk_kernel "
                    "(backward)",
                    "token-serial: st_forward_kernel, st_value_kernel, st_key_kernel"],
    }


def sclk_levels() -> list | None:
    """Current shader-clock level (MHz) of every card whose sysfs
    pp_dpm_sclk is readable (the line marked '*'), or None."""
    import glob
    import re

    out = []
    for path in sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")):
        try:
            text = Path(path).read_text()
        except OSError:
            continue
        for line in text.splitlines():
            if line.rstrip().endswith("*"):
                m = re.search(r"(\d+)\s*Mhz", line, re.I)
                if m:
                    out.append(int(m.group(1)))
    return out or None


def device_info(torch) -> dict:
    """Name and CU count of device 0, plus rocm-smi's current clock levels
    when the tool is present (the effective shader clock under the prefill
    kernel, from GRBM_GUI_ACTIVE, is in profiles/mfma_counters.json)."""
    import subprocess

    props = torch.cuda.get_device_properties(0)
    info = {"name": props.name, "arch": getattr(props, "gcnArchName", ""),
            "cus": props.multi_processor_count}
    # under a profiler (its library preloaded, the GPU initialised before
    # main) a child that execs another interpreter is refused: skip the tool
    profiled = any(k.startswith("ROCPROF") for k in os.environ) or \
        "rocprof" in os.environ.get("LD_PRELOAD", "")
    if profiled:
        return info
    try:
        out = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True,
                             timeout=20).stdout
        info["rocm_smi_clocks"] = [ln.split(":", 1)[1].strip() for ln in out.splitlines()
                                   if "clock level" in ln]
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def mfma_obj(w, kernel_ms: float):
    """Matrix-core use of the chunked kernel: issued bf16 MFMA flops (hi/lo
    split products included) over the launch time, against the dense bf16 peak."""
    import numpy as np

    lens = np.diff(w.cu_seqlens.cpu().numpy())
    chunks = int(((lens + 15) // 16).sum()) * w.num_heads
    flops = chunks * MFMA_PER_CHUNK * MFMA_FLOPS
    tf = flops / (kernel_ms * 1e-3) / 1e12
    out = {"issued_tflops": round(tf, 2), "peak_tflops": MFMA_PEAK_TFLOPS,
           "frac": round(tf / MFMA_PEAK_TFLOPS, 4), "instructions": chunks * MFMA_PER_CHUNK}
    # PMC-measured matrix-core use of the same kernel and workload
    # (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs), the MfmaUtil metric)
    path = ROOT / "profiles" / "mfma_counters.json"
    if path.exists():
        m = json.loads(path.read_text()).get("chunk64r_kernel<IoBF16>")
        if m is not None and m.get("workload") == w.name:
            out["measured_util"] = m["mfma_util"]
            out["measured_sclk_mhz"] = m["effective_sclk_mhz"]
            out["measured_source"] = ("profiles/mfma_counters.json: rocprofv3 --pmc "
                                      "SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE of the same "
                                      "kernel and workload; committed, not measured in this run")
    return out


def _frac(obj):
    return None if not obj else obj.get("frac")


def compact_line(result: dict) -> dict:
    """The printed JSON line: the headline fields, the headline kernel's
    roofline, timing, MFMA use and CPU baseline, then one short entry per
    further leg (ms, roofline fraction, kernel) so that the whole line stays
    a few KB.  The full tables go to --detail."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
            "roofline", "kernel_ms", "algorithmic_bytes", "timing")
    line = {k: result[k] for k in keep if k in result}
    if line.get("roofline") and line["roofline"].get("traffic_source"):
        line["roofline"] = dict(line["roofline"])
        line["roofline"]["traffic_source"] = "profiles/hbm_traffic.json (rocprofv3 PMC)"
    m = result.get("mfma")
    if m:
        line["mfma"] = {k: m[k] for k in ("issued_tflops", "peak_tflops", "frac",
                                          "measured_util") if k in m}
    cb = result.get("cpu_baseline")
    if cb:
        line["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    legs = {}
    d = result.get("decode")
    if d:
        legs["decode_cfg2"] = {"ms": d["kernel_ms"], "public_ms": d["ms_per_step"],
                               "frac": _frac(d["roofline"]), "kernel": d["kernel"]}
    d = result.get("decode_fp16_state")
    if d:
        legs["decode_fp16_state"] = {"ms": d["kernel_ms"], "frac": _frac(d["roofline"])}
    d = result.get("fp16_state_prefill")
    if d:
        legs["fp16_state_prefill_cfg1"] = {"ms": d["kernel_ms"], "public_ms": d["ms_per_step"],
                                           "frac": _frac(d["roofline"]), "kernel": d["kernel"],
                                           "workgroup_kernel_ms":
                                               d["forced_ms"]["serial_kernel<64,IoF16,StF16,8>"]}
    d = result.get("decode_graph")
    if d:
        legs["decode_graph"] = [{"workload": g["workload"], "graph_ms": g["graph_ms_per_step"],
                                 "eager_ms": g["eager_ms_per_step"]} for g in d]
    d = result.get("chunk_bf16_state")
    if d:
        legs["chunk_bf16_state_cfg1"] = {"ms": d.get("ms_per_step"),
                                         "frac": _frac(d.get("roofline"))}
    d = result.get("varlen_prefill")
    if d:
        legs["varlen_cfg3"] = {"ms": d["kernel_ms"], "public_ms": d["ms_per_step"],
                               "frac": _frac(d["roofline"]), "kernel": d["kernel"]}
    d = result.get("mid_length")
    if d:
        legs["mid_length_2048x100"] = {"ms": d["kernel_ms"], "frac": _frac(d["roofline"]),
                                       "kernel": d["kernel"]}
    d = result.get("long_context")
    if d:
        r = d["roofline"]
        legs["long_context_cfg4"] = {"ms": d["ms_per_step"], "frac": _frac(r),
                                     "traffic_over_algorithmic":
                                         round(r["traffic"] / d["algorithmic_bytes"], 3)
                                         if r.get("traffic") else None,
                                     "unsplit_ms": d["unsplit"]["ms_per_step"],
                                     "pieces": d["pieces"]}
    d = result.get("other_paths")
    if d:
        legs["other_paths_cfg1"] = {k: (v.get("kernel_ms") if isinstance(v, dict) else v)
                                    for k, v in d.items()
                                    if isinstance(v, dict) and "kernel_ms" in v}
    for key in ("pretrain_training", "statetune_training"):
        d = result.get(key)
        if d:
            legs[key] = {k: v for k, v in d.items()
                         if k.endswith("_ms") or k in ("forward_ms", "backward_ms")}
            for sub in ("chunked", "token_serial"):
                if isinstance(d.get(sub), dict):
                    legs[key][sub] = {k: v for k, v in d[sub].items() if k.endswith("_ms")}
            if isinstance(d.get("backward_roofline"), dict):
                legs[key]["backward_frac"] = d["backward_roofline"].get("frac")
    d = result.get("statetune_ragged")
    if d:
        legs["statetune_ragged_cfg1"] = {k: d[k] for k in ("chunked", "token_serial")}
    d = result.get("kk_gate_fused")
    if d:
        legs["kk_gate_fused_cfg1_fp16"] = {"two_stage_ms": d["two_stage"]["ms_per_step"],
                                           "fused_ms": d["fused"]["ms_per_step"],
                                           "readout_fused_ms":
                                               d["with_readout"]["fused"]["ms_per_step"]}
    d = result.get("layer_stages")
    if d:
        legs["layer_stages"] = {k: _frac(v["roofline"]) for k, v in d["kernels"].items()}
    line["device"] = {k: v for k, v in result.get("device", {}).items() if k != "rocm_smi_clocks"}
    line["legs"] = legs
    return line


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--settle", type=float, default=1.0,
                    help="after the warm-up steps, keep issuing untimed steps until this many "
                         "seconds have passed (clock ramp); reported in the line")
    ap.add_argument("--detail", default=None,
                    help="write the full result (every leg's tables) to this JSON file; the "
                         "printed line carries a compact summary")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode (config 2) leg")
    ap.add_argument("--cpu-sample-tokens", type=int, default=4096,
                    help="tokens per sequence in the CPU baseline sample")
    ap.add_argument("--no-train", action="store_true",
                    help="skip the training (forward + backward) leg")
    ap.add_argument("--only", choices=["prefill", "decode", "long", "mid", "train", "stages",
                                       "fp16"],
                    default=None,
                    help="run one leg only (profiling)")
    ap.add_argument("--config", type=int, default=1, choices=[1, 3, 4],
                    help="prefill workload (BASELINE config; the metric is quoted on 1)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (a known-size "
                         "kernel for scaling the HBM byte counters of a profile)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X only (one GPU per box); "
              "multi-GPU runs are not part of it", file=sys.stderr)
        return 2

    import torch

    import flashrwkv2_amd
    from flashrwkv2_amd import workloads

    if flashrwkv2_amd._C is None:
        print("bench.py: no GPU backend (flashrwkv2_amd._C is None)", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    result: dict = {}
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_probe_bytes"] = {"read": n * 4, "written": n * 4}
        del src, dst

    pre = None
    if args.only in (None, "prefill"):
        w1 = workloads.config(args.config, "cuda")
        pre = Runner(w1, torch, flashrwkv2_amd)
        sclk_before = sclk_levels()
        ms = pre.time_steps(args.steps, args.warmup, args.settle)
        kms = pre.time_kernel(args.steps)
        sclk_after = sclk_levels()
        bytes1 = algorithmic_bytes(w1.total_tokens, w1.num_heads, w1.state_indices.numel())
        result.update({
            "metric": METRIC,
            "value": round(w1.total_tokens / (ms * 1e-3), 1),
            "unit": "tokens/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms, 5),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (seeded, BASELINE config 1 distributions; inputs resident in HBM)",
            "config": {"workload": w1.name, **w1.info, "D": 64,
                       "io": "bf16", "state": "fp32",
                       "arithmetic": "bf16 MFMA on hi/lo split operands, fp32 accumulate",
                       "kernel": pre.kernel_name(),
                       "parallelism": "single GPU"},
            "roofline": roofline_obj(bytes1, kms, measured_traffic(pre.kernel_name(), w1.name)),
            "mfma": mfma_obj(w1, kms) if pre.kernel_name().startswith("chunk") else None,
            # the token-serial form's own roofline: recurrence-form flops
            # (5 x D x D FMA per token-head) over this kernel's time
            "valu_equivalent": {
                "achieved_tflops": round(w1.total_tokens * w1.num_heads * FLOPS_PER_TOKEN_HEAD
                                         / (kms * 1e-3) / 1e12, 2),
                "peak_tflops": VALU_FP32_PEAK_TFLOPS,
                "frac": round(w1.total_tokens * w1.num_heads * FLOPS_PER_TOKEN_HEAD
                              / (kms * 1e-3) / 1e12 / VALU_FP32_PEAK_TFLOPS, 4),
                "flops_per_token_head": FLOPS_PER_TOKEN_HEAD,
            },
            "kernel_ms": round(kms, 5),
            "algorithmic_bytes": bytes1,
            "timing": {"settle": pre.settle, "steps": pre.step_stats,
                       "public_over_kernel": round(ms / kms, 4),
                       "sclk_mhz_before_after": [sclk_before, sclk_after],
                       "public_path": "_C.tmix_wkv7_recurrent_fp32_from_decay_logits with a "
                                      "reused ticket (Python checks, METH_FASTCALL launch)"},
        })
    if args.only in (None, "decode") and not args.no_decode:
        w2 = workloads.config(2, "cuda")
        dec = Runner(w2, torch, flashrwkv2_amd)
        dms = dec.time_steps(max(args.steps, 50), args.warmup, min(args.settle, 0.3))
        dkms = dec.time_kernel(max(args.steps, 200))
        bytes2 = algorithmic_bytes(w2.total_tokens, w2.num_heads, w2.state_indices.numel())
        result["decode"] = {
            "workload": w2.name, "tokens_per_s": round(w2.total_tokens / (dms * 1e-3), 1),
            "ms_per_step": round(dms, 5), "kernel_ms": round(dkms, 5),
            "kernel_tokens_per_s": round(w2.total_tokens / (dkms * 1e-3), 1),
            "kernel": dec.kernel_name(),
            "roofline": roofline_obj(bytes2, dkms, measured_traffic(dec.kernel_name(), w2.name)),
            "algorithmic_bytes": bytes2,
        }
        # the same decode shape with fp16 tokens and the FP16 state pool
        # (8 KiB per (sequence, head)): infer_tmix_wkv7_recurrent_fp16_forward_varlen
        w3 = workloads.config(2, "cuda", dtype=torch.float16)
        f16_ms, f16_kms = time_fp16_state_decode(torch, flashrwkv2_amd, w3, max(args.steps, 50),
                                                 args.warmup)
        bytes3 = w3.total_tokens * w3.num_heads * BYTES_PER_TOKEN_HEAD + 2 * w3.state_indices.numel() * w3.num_heads * 64 * 64 * 2
        result["decode_fp16_state"] = {
            "workload": w3.name + "_fp16_state", "tokens_per_s": round(w3.total_tokens / (f16_ms * 1e-3), 1),
            "ms_per_step": round(f16_ms, 5), "kernel_ms": round(f16_kms, 5),
            "kernel": "decode64_f16s_kernel<IoF16>",
            "kernel_ms_note": "fr2_wkv7_recurrent_fp16_update alone; the public step also "
                              "launches the elapsed-state advance",
            "roofline": roofline_obj(bytes3, f16_kms), "algorithmic_bytes": bytes3,
        }
        # the same decode shape, and a small serving batch, as a captured
        # graph of consecutive steps on the graph-ticket path
        result["decode_graph"] = [
            time_graph_decode(torch, flashrwkv2_amd, workloads.config(2, "cuda", dtype=torch.float16)),
            time_graph_decode(torch, flashrwkv2_amd,
                              workloads.config(2, "cuda", dtype=torch.float16, batch=8)),
        ]
        if not result.get("metric"):
            result.update({"metric": METRIC, "value": result["decode"]["tokens_per_s"],
                           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
                           "warmup": args.warmup, "ms_per_step": round(dms, 5)})
    if args.only in (None, "prefill", "fp16") and args.config == 1:
        result["fp16_state_prefill"] = time_fp16_state_prefill(torch, flashrwkv2_amd,
                                                               max(4, args.steps // 4))
    if args.only in (None, "prefill") and args.config == 1 and pre is not None:
        result["chunk_bf16_state"] = time_chunk_bf16_state(torch, flashrwkv2_amd, pre.w,
                                                           max(5, args.steps // 2))
    if args.only in (None, "prefill") and args.config == 1 and pre is not None:
        result["other_paths"] = time_other_paths(torch, flashrwkv2_amd, pre.w, args.steps)
    if args.only in (None, "long") and args.config == 1:
        result["varlen_prefill"] = time_varlen(torch, flashrwkv2_amd, max(5, args.steps // 2))
    if args.only in (None, "long", "mid") and args.config == 1:
        result["mid_length"] = time_mid_length(torch, flashrwkv2_amd, max(5, args.steps // 4))
    if args.only in (None, "long") and args.config == 1:
        result["short_batches"] = time_short_batches(torch, flashrwkv2_amd, max(5, args.steps // 2))
        result["long_context"] = time_long_context(torch, flashrwkv2_amd, max(4, args.steps // 4))
    if args.only in (None, "train") and not args.no_train:
        wt = pre.w if (pre is not None and args.config == 1) else workloads.config(1, "cuda")
        result["pretrain_training"] = time_pretrain_training(torch, wt, max(3, args.steps // 4))
        result["statetune_training"] = time_statetune_training(torch, wt, max(3, args.steps // 4))
        result["statetune_ragged"] = time_statetune_ragged(torch, wt, max(3, args.steps // 4))
    if args.only in (None, "stages"):
        result["layer_stages"] = time_layer_stages(torch, 8 * 4096, 32)
        result["kk_gate_fused"] = time_kk_fused(torch, flashrwkv2_amd, max(5, args.steps // 2))
        result["kk_gate_fused_serving"] = time_kk_fused(torch, flashrwkv2_amd,
                                                        max(5, args.steps // 4), serving=True)
    result["device"] = device_info(torch)
    if pre is not None and not args.no_cpu and args.config == 1:
        threads = min(16, len(os.sched_getaffinity(0)) or 1)
        tps, dt, n_tok, reps = cpu_baseline(pre.w, threads, args.cpu_sample_tokens)
        result["cpu_baseline"] = {
            "value": round(tps, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"first {args.cpu_sample_tokens} tokens of each of the 8 config-1 "
                      f"sequences, all 32 heads ({n_tok} tokens x {reps} passes, {dt:.2f} s), fp32 C "
                      "recurrence (oracle/wkv7_oracle.c, OpenMP over sequence x head)",
            "cpu": cpu_info(),
        }
        result["cpu_baseline_plan"] = cpu_baseline_plan(threads)
    if args.detail:
        Path(args.detail).write_text(json.dumps(result, indent=1))
    print(json.dumps(compact_line(result)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
