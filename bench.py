#!/usr/bin/env python3
"""Benchmark of the k8v4 quantized paged-KV attention path on one MI355X.

One step = one decode/MTP-verify layer call (split-K kernel + merge kernel)
over the headline workload: 4 sequences x 131,072 cached tokens, 7 query
tokens each, 24 Q / 4 KV heads, head_dim 128, 64-token pages, random
non-contiguous block tables.  Prints ONE JSON line:

* ``value``: whole-step throughput in GB/s of algorithmic KV bytes
  (4 x 131,072 tokens x 816 B = 427,819,008 B per step), from the wall clock
  around exactly ``--steps`` steps bracketed by device synchronisations;
* ``roofline``: the split-K kernel inside full steps, timed with HIP events
  on the stream it runs on -- one recorded before each step, one the library
  records between its split and merge kernels -- over ``--steps`` steps run
  right after the wall-clock ones, against the 8 TB/s HBM peak
  (``kernel_us_back_to_back``: the same kernel launched alone, back to back,
  which starts while the previous launch's stores drain); ``traffic`` comes
  from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary when present;
* ``cpu_baseline``: the reference's PyTorch path restated in torch
  (oracle/torch_cpu.py) on every host core: the whole headline decode step,
  config 2's store and config 5's whole prefill chunk, plus config 1's shape
  through the pure-Python ``causal_gqa`` on one thread; the float64 oracle
  checks the GPU's headline output, the torch port the GPU's prefill output;
* ``step_graph_us`` and the configs' ``graph_us_*``: per-launch time from HIP
  graphs of back-to-back launches replayed between two events (median and
  min of several replays), which leaves out the host launch cost;
* ``configs``: microseconds per layer of the other workloads (store, short
  decode, MTP verify, mixed long context, prefill, the D=256 per-rank shape,
  four 256-dim KV heads, prefill at the D=256 per-rank shape).

Inputs are synthetic: fp16 N(0,1) K/V quantized into the cache by the store
kernel, fp16 N(0,1) queries.  Several copies of each cache are rotated from
step to step so that no step finds its pages in the 256 MB MALL.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO / "k8v4-xpu_amd"), str(REPO)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
METRIC = "K8V4 paged-decode HBM GB/s (% of peak) + µs/layer at 4 seqs×128K ctx"
TRAFFIC_PROFILE = REPO / "profiles" / "decode_split_kernel_headline_traffic.md"
PAGE = 64


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--splits", type=int, default=0, help="split-K work-groups (0 = library default)")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--only", default=None,
                    help="run only the config rows whose name contains this text (no headline; for profiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="with --only: also time the 1 GiB device copy that calibrates the byte counters")
    return ap.parse_args(argv)


# --------------------------------------------------------------------- HIP events
class HipEvents:
    """hipEvent_t helpers through the HIP runtime torch already loaded."""

    def __init__(self):
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise RuntimeError("the HIP runtime is not loaded")
        self.lib = ctypes.CDLL(path)
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self) -> int:
        ev = ctypes.c_void_p()
        rc = self.lib.hipEventCreate(ctypes.byref(ev))
        if rc != 0:
            raise RuntimeError("hipEventCreate failed (%d)" % rc)
        return ev.value

    def record(self, ev: int, stream: int) -> None:
        rc = self.lib.hipEventRecord(ctypes.c_void_p(ev), ctypes.c_void_p(stream))
        if rc != 0:
            raise RuntimeError("hipEventRecord failed (%d)" % rc)

    def ms(self, a: int, b: int) -> float:
        self.lib.hipEventSynchronize(ctypes.c_void_p(b))
        out = ctypes.c_float()
        rc = self.lib.hipEventElapsedTime(ctypes.byref(out), ctypes.c_void_p(a), ctypes.c_void_p(b))
        if rc != 0:
            raise RuntimeError("hipEventElapsedTime failed (%d)" % rc)
        return float(out.value)

    def destroy(self, ev: int) -> None:
        self.lib.hipEventDestroy(ctypes.c_void_p(ev))


# --------------------------------------------------------------------- workloads
class DecodeWorkload:
    """``copies`` independent caches of one decode shape in one page pool."""

    def __init__(self, ops, torch, *, lengths, q_len, hkv, head_dim, copies, seed,
                 pool_pages_per_copy=None, shared_prefix_pages=0, splits=0):
        from k8v4_v030.layout import PageLayout
        from k8v4_v030.cache_views import bind_regions

        self.torch, self.ops = torch, ops
        self.lengths = list(lengths)
        self.batch = len(self.lengths)
        self.q_len, self.hkv, self.head_dim = q_len, hkv, head_dim
        self.layout = PageLayout(hkv, head_dim)
        pages = [-(-n // PAGE) for n in self.lengths]
        self.width = max(pages)
        unique = shared_prefix_pages + sum(max(0, p - shared_prefix_pages) for p in pages)
        per_copy = max(pool_pages_per_copy or 0, unique)
        self.num_pages = per_copy * copies
        gen = torch.Generator().manual_seed(seed)
        self.raw = torch.empty(self.num_pages * self.layout.page_bytes, dtype=torch.int8, device="cuda")
        self.views = bind_regions(self.raw, self.layout)
        fill_pool(ops, torch, self.views, self.num_pages, hkv, head_dim, seed)
        tables = []
        for c in range(copies):
            perm = torch.randperm(per_copy, generator=gen) + c * per_copy
            table = torch.zeros((self.batch, self.width), dtype=torch.int32)
            shared = perm[:shared_prefix_pages]
            cur = shared_prefix_pages
            for b, n in enumerate(pages):
                s = min(n, shared_prefix_pages)
                table[b, :s] = shared[:s].to(torch.int32)
                table[b, s:n] = perm[cur : cur + n - s].to(torch.int32)
                cur += n - s
            tables.append(table.to("cuda"))
        self.tables = tables
        self.seq_lens = torch.tensor(self.lengths, dtype=torch.int32, device="cuda")
        qgen = torch.Generator(device="cuda").manual_seed(seed + 1)
        self.q = torch.randn((self.batch * q_len, 6 * hkv, head_dim), generator=qgen,
                             dtype=torch.float16, device="cuda")
        self.out = torch.empty_like(self.q)
        nbytes = ops.attn_workspace_bytes(self.batch, self.width, 1, q_len, hkv, head_dim, splits)
        self.ws = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
        self.splits = splits
        # Bytes the step reads (a shared prefix page once per sequence that reads it),
        # and the distinct bytes behind them (each shared page counted once).
        self.kv_bytes = sum(self.lengths) * self.layout.bytes_per_token
        shared_tokens = shared_prefix_pages * PAGE
        self.unique_kv_bytes = (min(max(self.lengths), shared_tokens)
                                + sum(max(0, n - shared_tokens) for n in self.lengths)) * self.layout.bytes_per_token
        v = self.views
        self.calls = [
            ops.bind_int8k_int4v_attn_batch(
                self.q, None, None, v["k"], v["k_scale"], v["v"], v["v_scale"], v["v_zero"], t,
                self.seq_lens, None, self.ws, None, None, None, self.out, q_len, 1, num_splits=splits)
            for t in self.tables
        ]

    def launch(self, i: int, split_done=None, stages=3):
        self.calls[i % len(self.calls)](split_done_event=split_done, stages=stages)


def fill_pool(ops, torch, views, num_pages, hkv, head_dim, seed, chunk=65536):
    """Every page of the pool gets quantized fp16 N(0,1) tokens from the store kernel."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    total = num_pages * PAGE
    for s in range(0, total, chunk):
        e = min(total, s + chunk)
        k = torch.randn((e - s, hkv, head_dim), generator=gen, dtype=torch.float16, device="cuda")
        v = torch.randn((e - s, hkv, head_dim), generator=gen, dtype=torch.float16, device="cuda")
        slots = torch.arange(s, e, dtype=torch.int64, device="cuda")
        ops.kv_store_paged(k, v, slots, views["k"], views["k_scale"], views["v"], views["v_scale"], views["v_zero"])


class StoreWorkload:
    """4 x 4,224 new tokens quantized into a 16,384-page cache (1% entries x20)."""

    def __init__(self, ops, torch, *, copies, seed):
        from k8v4_v030.layout import PageLayout
        from k8v4_v030.cache_views import bind_regions

        self.torch, self.ops = torch, ops
        hkv, d, seqs, chunk = 4, 128, 4, 4224
        self.layout = PageLayout(hkv, d)
        self.num_pages = 16384
        self.raw = torch.zeros(self.num_pages * self.layout.page_bytes, dtype=torch.int8, device="cuda")
        self.views = bind_regions(self.raw, self.layout)
        gen = torch.Generator().manual_seed(seed)
        dgen = torch.Generator(device="cuda").manual_seed(seed)
        ntok = seqs * chunk
        self.inputs = []
        for _ in range(copies):
            kv = []
            for _ in range(2):
                x = torch.randn((ntok, hkv, d), generator=dgen, dtype=torch.float16, device="cuda")
                hit = torch.rand(x.shape, generator=dgen, device="cuda") < 0.01
                kv.append(torch.where(hit, x * 20, x))
            pages = torch.randperm(self.num_pages, generator=gen)[: seqs * chunk // PAGE]
            t = torch.arange(ntok)
            slots = pages[t // PAGE] * PAGE + t % PAGE
            self.inputs.append(ops.bind_kv_store_paged(kv[0], kv[1], slots.to("cuda"), self.views["k"],
                                                       self.views["k_scale"], self.views["v"],
                                                       self.views["v_scale"], self.views["v_zero"]))
        self.ntok = ntok
        self.algo_bytes = ntok * hkv * d * 2 * 2 + ntok * 8 + ntok * self.layout.bytes_per_token

    def launch(self, i: int, split_done=None, stages=3):
        self.inputs[i % len(self.inputs)]()


class PrefillWorkload:
    """A 4,224-token query chunk over 131,072 cached tokens plus itself (one sequence)."""

    def __init__(self, ops, torch, *, cached=131072, chunk=4224, hkv=4, head_dim=128, seed=1005):
        import math

        from k8v4_v030.cache_views import bind_regions
        from k8v4_v030.layout import PageLayout

        self.layout = PageLayout(hkv, head_dim)
        self.seq_len, self.q_len = cached + chunk, chunk
        pages = -(-self.seq_len // PAGE)
        self.num_pages = pages
        self.raw = torch.empty(pages * self.layout.page_bytes, dtype=torch.int8, device="cuda")
        self.views = bind_regions(self.raw, self.layout)
        # The chunk's own K/V go through the store kernel like the cached prefix.
        fill_pool(ops, torch, self.views, pages, hkv, head_dim, seed)
        gen = torch.Generator().manual_seed(seed)
        self.row = torch.randperm(pages, generator=gen).to(torch.int32).to("cuda")
        qgen = torch.Generator(device="cuda").manual_seed(seed + 1)
        self.q = torch.randn((chunk, 6 * hkv, head_dim), generator=qgen, dtype=torch.float16, device="cuda")
        self.out = torch.empty_like(self.q)
        v = self.views
        self.call = ops.bind_prefill_paged(self.q, v["k"], v["k_scale"], v["v"], v["v_scale"], v["v_zero"],
                                           self.row, self.seq_len, 1, 1.0 / math.sqrt(head_dim), self.out)
        # Unmasked (query, key) pairs: query j sees cached + j + 1 keys.
        pairs = chunk * (cached + 1) + chunk * (chunk - 1) // 2
        self.flops = pairs * 6 * hkv * 4 * head_dim

    def launch(self, i: int, split_done=None, stages=3):
        self.call()


# --------------------------------------------------------------------- timing
def progress(msg: str) -> None:
    print("[bench] " + msg, file=sys.stderr, flush=True)


def synchronize(torch):
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        torch.distributed.barrier()
    torch.cuda.synchronize()


def warm_clocks(torch, work, seconds=2.0):
    """Run untimed steps until the GPU has been busy for ``seconds``.

    Measured on this part: a timed region that starts cold reads ~8% slower
    than the same region after two seconds of load (clocks ramp up)."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            work.launch(i)
            i += 1
        synchronize(torch)


def timed_wall(torch, work, steps, warmup):
    """Wall-clock seconds of exactly ``steps`` launches after ``warmup`` untimed ones."""
    warm_clocks(torch, work)
    for i in range(warmup):
        work.launch(i)
    synchronize(torch)
    t0 = time.perf_counter()
    for i in range(steps):
        work.launch(warmup + i)
    synchronize(torch)
    return time.perf_counter() - t0


def kernel_us(torch, hip, work, stages, steps, warmup):
    """Average microseconds per launch of one decode stage, launched back to back
    between two events on its stream (1 = split-K kernel, 2 = merge kernel)."""
    stream = int(torch.cuda.current_stream().cuda_stream)
    for i in range(warmup):
        work.launch(i, stages=stages)
    synchronize(torch)
    a, b = hip.create(), hip.create()
    hip.record(a, stream)
    for i in range(steps):
        work.launch(warmup + i, stages=stages)
    hip.record(b, stream)
    us = 1e3 * hip.ms(a, b) / steps
    hip.destroy(a)
    hip.destroy(b)
    return us


def split_in_step_us(torch, hip, work, steps, warmup):
    """Average microseconds of the split-K kernel inside full steps (split +
    merge): an event recorded on the launch stream before each step and one
    the library records between its two kernels (``split_done``)."""
    stream = int(torch.cuda.current_stream().cuda_stream)
    for i in range(warmup):
        work.launch(i)
    synchronize(torch)
    evs = [(hip.create(), hip.create()) for _ in range(steps)]
    for i, (a, b) in enumerate(evs):
        hip.record(a, stream)
        work.launch(warmup + i, split_done=b)
    synchronize(torch)
    us = 1e3 * sum(hip.ms(a, b) for a, b in evs) / steps
    for a, b in evs:
        hip.destroy(a)
        hip.destroy(b)
    return us


def graph_us(torch, work, launches=20, replays=10, reps=7):
    """Per-launch microseconds from a HIP graph of ``launches`` back-to-back
    launches (rotating the work's input copies), replayed ``replays`` times
    between two events, ``reps`` times: (median, min).  No host launch cost."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(launches):
            work.launch(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(launches):
            work.launch(i)
    for _ in range(3):
        graph.replay()
    synchronize(torch)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per = []
    for _ in range(reps):
        a.record()
        for _ in range(replays):
            graph.replay()
        b.record()
        synchronize(torch)
        per.append(1e3 * a.elapsed_time(b) / (replays * launches))
    del graph
    per.sort()
    return per[len(per) // 2], per[0]


def copy_peak_gbs(torch, hip, nbytes=1 << 30, reps=20):
    """Read+write GB/s of a plain device copy (the calibration kernel for byte counters)."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)

    class _Copy:
        def launch(self, i, split_done=None, stages=3):
            dst.copy_(src)

    us = kernel_us(torch, hip, _Copy(), 3, reps, 3)
    return 2 * nbytes / (us * 1e-6) / 1e9


def traffic_from_profile():
    """HBM bytes per split-kernel launch from the committed rocprofv3 PMC summary."""
    if not TRAFFIC_PROFILE.is_file():
        return None
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1].strip())
    return None


# --------------------------------------------------------------------- CPU baseline
def host_cpu():
    """(logical cores, CPU model name) of this host."""
    model = "unknown"
    try:
        import subprocess

        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except Exception:  # noqa: BLE001 -- the model name is informational
        pass
    return os.cpu_count() or 1, model


def median_seconds(fn, reps=3, warmup=1):
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline(torch, work, store_work=None, prefill_work=None):
    """The reference's PyTorch path (oracle/torch_cpu.py) on every host core.

    decode: the whole headline step (4 x 131,072 tokens, q = 7) -- gather and
    dequantize, int8 query rows, fp32 attention; store: config 2's 16,896 tokens
    quantized into the cache (both median of 3 after one warm-up); prefill:
    config 5's whole chunk over all 135,296 keys (key-tiled online softmax), once;
    config 1's shape through the pure-Python ``causal_gqa``, one thread.
    The float64 oracle checks the GPU's headline output on the same cache."""
    import numpy as np

    from oracle import attention, paged, torch_cpu

    cores, model = host_cpu()
    torch.set_num_threads(cores)
    work.launch(0)  # copy 0, whose tables the CPU reads
    torch.cuda.synchronize()
    geom = paged.Geometry(work.hkv, work.head_dim)
    raw_pages = work.raw.view(work.num_pages, work.layout.page_bytes)
    # The sequences' pages, gathered into one compact host cache with an identity-like table.
    tables = []
    blobs = []
    base = 0
    for b, n in enumerate(work.lengths):
        pages = -(-n // PAGE)
        blobs.append(raw_pages.index_select(0, work.tables[0][b, :pages].long()).view(torch.uint8).cpu())
        tables.append(torch.arange(base, base + pages, dtype=torch.int64))
        base += pages
    raw = torch.cat([x.reshape(-1) for x in blobs])
    views = torch_cpu.region_views(raw, geom)
    table = torch.nn.utils.rnn.pad_sequence(tables, batch_first=True)
    q = work.q.cpu()
    sec = median_seconds(lambda: torch_cpu.decode(views, q, table, work.lengths, work.q_len))
    gpu = work.out.double().cpu().numpy()
    blob = raw.numpy()
    err = 0.0
    for b, n in enumerate(work.lengths):
        rows = slice(b * work.q_len, (b + 1) * work.q_len)
        want = attention.decode_attention(q[rows].numpy(), blob, geom, table[b : b + 1].numpy(), [n], work.q_len)
        err = max(err, float(np.abs(gpu[rows] - want).max()))
    out = {
        "value": round(work.kv_bytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "cpu_model": model,
        "kind": "port",
        "sample": "the whole headline step on the host: torch restatement of the reference's CPU path "
                  "(oracle/torch_cpu.py decode: gather + dequantize %d x %d tokens, int8 query rows, fp32 "
                  "attention over 24 Q / 4 KV heads, D=128); median of 3 after 1 warm-up, %d threads"
                  % (work.batch, work.lengths[0], cores),
        "seconds": round(sec, 3),
        "us_per_layer": round(sec * 1e6, 1),
        "gpu_vs_float64_oracle_max_abs_err": err,
    }
    if store_work is not None:
        out["store"] = cpu_store_baseline(torch, store_work, torch_cpu, geom)
    if prefill_work is not None:
        out["prefill"] = cpu_prefill_baseline(torch, prefill_work, torch_cpu)
    out["config1_scalar"] = cpu_scalar_baseline()
    return out


def cpu_scalar_baseline():
    """Config 1's shape (1 x 2,048 tokens, q = 1, 24 Q / 4 KV heads, D = 128)
    through the pure-Python restatement of the reference's ``causal_gqa``
    (oracle/scalar.py; reference oracle.py:140-162), which quantizes the K and V
    rows itself: one thread, median of 3 after one warm-up, uniform rows."""
    from oracle import scalar

    seq, q_len, hq, hkv, dim = 2048, 1, 24, 4, 128
    key = scalar.deterministic_rows(seq, hkv, 1, dim)
    value = scalar.deterministic_rows(seq, hkv, 2, dim)
    query = scalar.deterministic_rows(q_len, hq, 3, dim)
    sec = median_seconds(lambda: scalar.causal_gqa(query, key, value, seq, q_len))
    kv_bytes = seq * hkv * (dim + dim // 2 + 12)
    return {"value": round(kv_bytes / sec / 1e9, 6), "unit": "GB/s", "cores": 1, "kind": "port",
            "seconds": round(sec, 3), "us_per_layer": round(sec * 1e6, 1),
            "sample": "config 1's shape through the pure-Python causal_gqa (quantizes 2,048 x 4 K and V rows, "
                      "then int8-Q attention for 24 heads), one thread, median of 3 after 1 warm-up"}


def cpu_store_baseline(torch, w, torch_cpu, geom):
    """Config 2 on the host: quantize 4 x 4,224 tokens into a 16,384-page cache."""
    call = w.inputs[0]
    k, v, slots = (t.cpu() for t in call._keep[:3])
    raw = torch.zeros(w.num_pages * w.layout.page_bytes, dtype=torch.uint8)
    views = torch_cpu.region_views(raw, geom)
    sec = median_seconds(lambda: torch_cpu.store(views, k, v, slots))
    return {"value": round(w.algo_bytes / sec / 1e9, 3), "unit": "GB/s", "us_per_layer": round(sec * 1e6, 1),
            "sample": "config 2 whole: %d tokens x 4 KV heads quantized (float64 rule) into the paged cache"
                      % w.ntok}


def cpu_prefill_baseline(torch, w, torch_cpu):
    """Config 5's whole chunk (4,224 query tokens over all 135,296 keys) on the
    host, once (about 17 s on 16 cores); the GPU's output of the same chunk is
    compared with it."""
    from oracle import paged

    geom = paged.Geometry(w.layout.hkv, w.layout.head_dim)
    raw = w.raw.view(torch.uint8).cpu()
    views = torch_cpu.region_views(raw, geom)
    q = w.q.cpu()
    row = w.row.cpu()
    w.launch(0)
    torch.cuda.synchronize()
    gpu = w.out.float().cpu()
    t0 = time.perf_counter()
    want = torch_cpu.prefill(views, q, row, w.seq_len, 1.0 / math.sqrt(w.layout.head_dim))
    sec = time.perf_counter() - t0
    return {"value": round(w.flops / sec / 1e12, 4), "unit": "TFLOP/s", "seconds": round(sec, 3),
            "us_per_layer": round(sec * 1e6, 0),
            "gpu_vs_cpu_port_max_abs_err": float((gpu - want).abs().max()),
            "sample": "the whole chunk: %d query tokens over all %d keys, one run (key tiles of 16,384, row groups "
                      "of 256, fp32)" % (w.q_len, w.seq_len)}


# --------------------------------------------------------------------- configs
def config_rows(torch, hip, ops, steps, warmup, only=None):
    rows = {}

    def want(name):
        return only is None or only in name

    def decode_row(name, lengths, q_len, copies, seed, hkv=4, head_dim=128, **kw):
        if not want(name):
            return
        w = DecodeWorkload(ops, torch, lengths=lengths, q_len=q_len, hkv=hkv, head_dim=head_dim,
                           copies=copies, seed=seed, **kw)
        warm_clocks(torch, w, 1.0)
        us = kernel_us(torch, hip, w, 3, steps, warmup)
        g_med, g_min = graph_us(torch, w)
        rows[name] = {
            "us_per_layer": round(us, 2),
            "graph_us_median": round(g_med, 2),
            "graph_us_min": round(g_min, 2),
            "split_kernel_us": round(kernel_us(torch, hip, w, 1, steps, warmup), 2),
            "merge_kernel_us": round(kernel_us(torch, hip, w, 2, steps, warmup), 2),
            "kv_bytes": w.kv_bytes,
            "GBps": round(w.kv_bytes / (us * 1e-6) / 1e9, 1),
            "pct_of_hbm_peak": round(100 * w.kv_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
            "cache_copies_rotated": copies,
        }
        if w.unique_kv_bytes != w.kv_bytes:
            # A shared prefix is read once per sequence in the same step: the rate
            # on distinct bytes sits beside the rate on bytes read.
            rows[name].update({
                "unique_kv_bytes": w.unique_kv_bytes,
                "GBps_unique": round(w.unique_kv_bytes / (us * 1e-6) / 1e9, 1),
                "pct_of_hbm_peak_unique": round(100 * w.unique_kv_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
            })
        del w
        torch.cuda.empty_cache()
        progress("%s: %.2f us/layer" % (name, us))

    decode_row("1_decode_ctx2048_q1", [2048], 1, copies=128, seed=1001, pool_pages_per_copy=64)
    if want("2_store_4x4224_tokens"):
        w = StoreWorkload(ops, torch, copies=8, seed=1002)
        warm_clocks(torch, w, 1.0)
        us = kernel_us(torch, hip, w, 3, steps, warmup)
        g_med, g_min = graph_us(torch, w)
        rows["2_store_4x4224_tokens"] = {
            "us_per_layer": round(us, 2),
            "graph_us_median": round(g_med, 2),
            "graph_us_min": round(g_min, 2),
            "algorithmic_bytes": w.algo_bytes,
            "GBps": round(w.algo_bytes / (us * 1e-6) / 1e9, 1),
            "pct_of_hbm_peak": round(100 * w.algo_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
            "input_copies_rotated": 8,
        }
        progress("2_store_4x4224_tokens: %.2f us/layer" % us)
        del w
        torch.cuda.empty_cache()
    decode_row("3_mtp_verify_4x8192_q7", [8192] * 4, 7, copies=12, seed=1003, pool_pages_per_copy=1024)
    decode_row("4_mixed_long_q7", [2048, 32768, 131072, 200000], 7, copies=3, seed=1004,
               shared_prefix_pages=1024)
    def prefill_row(name, hkv, head_dim, dtype, graph=True):
        if not want(name):
            return
        w = PrefillWorkload(ops, torch, hkv=hkv, head_dim=head_dim)
        warm_clocks(torch, w, 1.0)
        us = kernel_us(torch, hip, w, 3, max(5, steps // 10), 2)
        tflops = w.flops / (us * 1e-6) / 1e12
        rows[name] = {"us_per_layer": round(us, 1)}
        if graph:
            g_med, g_min = graph_us(torch, w, launches=2, replays=2, reps=3)
            rows[name].update({"graph_us_median": round(g_med, 1), "graph_us_min": round(g_min, 1)})
        rows[name].update({
            "algorithmic_flops": w.flops,
            "TFLOPs": round(tflops, 1),
            "mfma_peak_TFLOPs": MFMA_F16_PEAK_TFLOPS,
            "mfma_utilization": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "dtype": dtype,
        })
        del w
        torch.cuda.empty_cache()
        progress("%s: %.1f us/layer, %.1f TFLOP/s" % (name, us, tflops))

    prefill_row("5_prefill_4224_over_131072", 4, 128,
                "f16 MFMA (fp16 tiles: K code x k_scale, V (nibble - v_zero) x v_scale / 16), f32 accumulation")
    decode_row("reference_shape_d256_hkv2_ctx127853_q7", [127853], 7, copies=4, seed=1007,
               hkv=2, head_dim=256)
    decode_row("d256_hkv4_4x32768_q7", [32768] * 4, 7, copies=3, seed=1008, hkv=4, head_dim=256)
    prefill_row("prefill_d256_hkv2_4224_over_131072", 2, 256,
                "f16 MFMA (fp16 tiles: K code x k_scale, V nibbles as fp16 subnormals), f32 accumulation",
                graph=False)
    return rows


# --------------------------------------------------------------------- main
def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(got --gpus %d)" % args.gpus, file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    from k8v4_v030.ops_api import ops

    o = ops()
    hip = HipEvents()
    if args.only:
        rows = config_rows(torch, hip, o, min(args.steps, 100), min(args.warmup, 10), only=args.only)
        line = {"configs": rows}
        if args.calibrate_copy:
            line["copy_peak_GBps"] = round(copy_peak_gbs(torch, hip), 1)
        print(json.dumps(line), flush=True)
        return 0
    B, ctx, q_len = 4, 131072, 7
    work = DecodeWorkload(o, torch, lengths=[ctx] * B, q_len=q_len, hkv=4, head_dim=128, copies=3,
                          seed=1006, splits=args.splits)
    progress("headline cache filled")
    wall = timed_wall(torch, work, args.steps, args.warmup)
    ms_per_step = 1e3 * wall / args.steps
    gbs = work.kv_bytes / (wall / args.steps) / 1e9

    split_us = split_in_step_us(torch, hip, work, args.steps, args.warmup)
    step_graph = graph_us(torch, work)
    split_b2b_us = kernel_us(torch, hip, work, 1, args.steps, args.warmup)
    merge_us = kernel_us(torch, hip, work, 2, args.steps, args.warmup)
    achieved = work.kv_bytes / (split_us * 1e-6) / 1e9
    copy_gbs = copy_peak_gbs(torch, hip)
    progress("headline: %.2f us/layer, split kernel %.2f us" % (1e3 * ms_per_step, split_us))

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 QK (i32 acc) + f16 PV (f32 acc)",
        "data": "synthetic",
        "config": {
            "workload": "paged decode / MTP verify: 4 seqs x 131072 cached tokens, 7 query tokens each, "
                        "24 Q / 4 KV heads, head_dim 128, 64-token int8-K/int4-V pages, random block tables",
            "batch": B, "context": ctx, "q_len": q_len, "hq": 24, "hkv": 4, "head_dim": 128,
            "page_tokens": PAGE, "kv_bytes_per_step": work.kv_bytes, "cache_copies_rotated": 3,
            "parallelism": "single GPU",
        },
        "us_per_layer": round(1e3 * ms_per_step, 2),
        "step_graph_us": {"median": round(step_graph[0], 2), "min": round(step_graph[1], 2),
                          "launches": "hipGraph of 20 steps, 10 replays x 7"},
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "roofline": {
            "kernel": "decode_split_kernel",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profile(),
            "algorithmic_bytes_per_launch": work.kv_bytes,
            "kernel_us": round(split_us, 2),
            "kernel_timing": "inside full steps: HIP events before each step and between split and merge",
            "kernel_us_back_to_back": round(split_b2b_us, 2),
            "merge_kernel_us": round(merge_us, 2),
            "copy_peak_GBps": round(copy_gbs, 1),
            "frac_of_copy_peak": round(achieved / copy_gbs, 4),
        },
    }
    if not args.no_cpu:
        store_w = StoreWorkload(o, torch, copies=1, seed=1002)
        prefill_w = PrefillWorkload(o, torch)
        line["cpu_baseline"] = cpu_baseline(torch, work, store_w, prefill_w)
        progress("cpu baseline: decode %.1f s" % line["cpu_baseline"]["seconds"])
        del store_w, prefill_w
    del work
    torch.cuda.empty_cache()
    if not args.no_configs:
        line["configs"] = config_rows(torch, hip, o, min(args.steps, 100), min(args.warmup, 10))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
