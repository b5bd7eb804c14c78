"""Benchmark of the paged decode hot path on one MI355X.

One step = one fused KV-append + paged decode-attention launch
(``mt_paged_decode_split``: the decode of ``mt_paged_decode_batch`` with the
rows visited longest first) over one batch of config 2: B = 64
requests, contexts L ~ U{128..1024}, 12 heads, head_dim 64, page 16, fp16 K/V
with fp32 accumulation, an 8192-page pool shuffled from the seed. Inputs are
resident in HBM before the timed region. To measure cold-cache HBM bandwidth,
steps rotate over ``--pools`` disjoint copies of the pool, tables and Q/K/V
(6 x ~113 MB touched per cycle, beyond the 256 MB Infinity Cache).

Prints one JSON line: the op-level rate (B requests per step / mean step time
from HIP events around the K timed steps; one layer's fused append + attention,
not a whole-model rate), the roofline of the decode kernel (algorithmic bytes
per launch / mean launch time vs 8 TB/s) and the CPU baseline (the C
restatement in oracle/, OpenMP on the host cores, on a bounded sample of the
same workload); then, under ``config1`` and ``e2e``, config 1's launch time
beside its CPU time and the end-to-end decode tokens/s of configs 3
(DistilGPT-2 fp16 trace, by the reference's formula and over busy steps) and 4
(GPT-2-medium bf16 steady state, ms per decode step), each with its CPU
baseline. ``--no-e2e`` skips those.
"""
import argparse
import ctypes as ct
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from minitorch_amd.runtime import runtime, CudaEvent, P, I, Z  # noqa: E402
from minitorch_amd import paged_ops  # noqa: E402
from minitorch_amd.workloads import config2_case, DevicePagedCase  # noqa: E402

PEAK_HBM_GBS = 8000.0
PEAK_MFMA_TFLOPS = 2500.0  # dense fp16/bf16 matrix cores
METRIC = 'decode tokens/s (1 GPU) + paged-attn achieved HBM GB/s as % of MI355X peak'


def algorithmic_bytes(case):
    """Minimum HBM traffic of one append + attention launch.

    bytes_append = B*H*D*2*(s_in + s_kv)
    bytes_attn   = sum_i 2*L_i*H*D*s_kv + B*H*D*(s_q + s_o) + sum_i 4*ceil(L_i/P) + 4*B
    """
    s = 4 if case.dtype == 'float32' else 2
    B, H, D, Pg = case.batch, case.heads, case.dim, case.page_size
    L = case.lengths.astype(np.int64)
    append = B * H * D * 2 * (s + s)
    attn = int((2 * L * H * D * s).sum()) + B * H * D * (s + s) + int((4 * ((L + Pg - 1) // Pg)).sum()) + 4 * B
    return append + attn


def measured_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (calibrated against a copy of known size), or None."""
    path = os.path.join(ROOT, 'profiles', 'decode_config2_fp16_hbm_traffic.md')
    try:
        for line in open(path):
            if line.startswith('traffic_bytes_per_launch:'):
                return int(line.split(':')[1])
    except OSError:
        pass
    return None


def host_cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return None


def timed_steps(run, seconds, min_steps=10):
    """Per-step wall times of ``run()`` repeated for ``seconds`` (at least
    ``min_steps`` steps) after one untimed warm-up step."""
    run()
    times, t_end = [], time.perf_counter() + seconds
    while len(times) < min_steps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return np.asarray(times)


def cpu_baseline(case, seconds):
    """The C oracle's decode step (append + attention, fp32 arithmetic, OpenMP
    over (request, head)) on the host cores: the median step time on up to 16
    threads over ``seconds``, and on one thread over half as long."""
    try:
        from oracle import c_oracle
        lib = c_oracle.library()
    except Exception as error:  # the oracle library is optional on the GPU box
        return dict(value=None, unit='tokens/s', cores=None, kind='port', sample=f'unavailable: {error}')
    host = c_oracle.HostCase(case)
    threads = min(os.cpu_count() or 1, 16)
    many = timed_steps(lambda: host.run(lib, threads), seconds)
    one = timed_steps(lambda: host.run(lib, 1), seconds / 2)
    rate = lambda t: case.batch / float(np.median(t))
    return dict(value=rate(many), unit='tokens/s', cores=threads, kind='port',
                sample=f'median of {len(many)} steps of config 2 (B=64, same seed, {many.sum():.1f} s), fp32 '
                       f'arithmetic on fp16 pages, OpenMP over (request, head)',
                single_core=dict(value=rate(one), cores=1, steps=len(one)),
                host=dict(nproc=os.cpu_count(), cpu_model=host_cpu_model()))


def ragged_cpu_baseline(case, seconds):
    """The C oracle's decode step (append + attention, fp32 arithmetic) on a
    device-built ragged case, downloaded to the host: median step time on up
    to 16 threads over ``seconds`` and on one thread (at least 10 steps each)."""
    try:
        from oracle import c_oracle
        lib = c_oracle.library()
    except Exception as error:  # the oracle library is optional on the GPU box
        return dict(value=None, unit='tokens/s', cores=None, kind='port', sample=f'unavailable: {error}')
    image = case.pool.download(np.uint16 if case.dtype != 'float32' else np.float32)
    q, k, v = (t.raw_numpy() for t in (case.q, case.k, case.v))
    slabs = np.array([image.ctypes.data + s * case.slab_bytes for s in range(case.num_slabs)], np.uint64)
    table = np.ascontiguousarray(case.table_host, np.int32)
    offsets = (case.lengths - 1).astype(np.int32)
    out = np.zeros_like(q)
    code = c_oracle.CODES[case.dtype]

    def run(threads):
        status = lib.oracle_paged_decode_batch(out.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                               slabs.ctypes.data, table.ctypes.data, offsets.ctypes.data,
                                               case.batch, case.heads, case.dim, case.page_size,
                                               case.pages_per_slab, case.num_slabs, case.columns, 0, 1, code,
                                               threads)
        if status:
            raise RuntimeError(f'oracle_paged_decode_batch returned {status}')

    threads = min(os.cpu_count() or 1, 16)
    many = timed_steps(lambda: run(threads), seconds)
    one = timed_steps(lambda: run(1), seconds / 2)
    rate = lambda t: case.batch / float(np.median(t))
    return dict(value=rate(many), unit='tokens/s', cores=threads, kind='port',
                sample=f'median of {len(many)} full config-5 steps (B=512, H=25, P={case.page_size}, same '
                       f'hash-filled pool downloaded from the device, {many.sum():.1f} s), fp32 arithmetic on '
                       f'{case.dtype} pages, OpenMP over (request, head)',
                single_core=dict(value=rate(one), cores=1, steps=len(one)),
                host=dict(nproc=os.cpu_count(), cpu_model=host_cpu_model()))


def pattern_ceiling(case, devs, steps, warmup):
    """Bandwidth of the decode step's K/V access pattern alone: every (row,
    head, page) K and V page-head chunk (P*D*s bytes, randomly placed by the
    shuffled table) read by mt_chunk_read, a kernel with no address
    arithmetic, math or merge, at the decode's grid and at a large grid; and,
    for reference, the same number of bytes read sequentially (consecutive
    chunks of rotated buffers) by the same kernel in one launch."""
    from minitorch_amd.runtime import RawDeviceBuffer
    rt = runtime()
    s = 2 if case.dtype != 'float32' else 4
    H, Pg, D, pps = case.heads, case.page_size, case.dim, case.pages_per_slab
    chunk = Pg * D * s
    plane = pps * H * Pg * D * s
    lists = []
    for d in devs:
        addrs = []
        for b in range(case.batch):
            pages = case.table[b, :(int(case.lengths[b]) + Pg - 1) // Pg]
            for h in range(H):
                for p in pages:
                    base = d.pool.ptr + (int(p) // pps) * case.slab_bytes + ((int(p) % pps) * H + h) * chunk
                    addrs += [base, base + plane]
        buf = RawDeviceBuffer(8 * len(addrs))
        buf.upload(np.array(addrs, np.uint64))
        lists.append((buf, len(addrs)))
    sink = RawDeviceBuffer(4)
    f = rt.lib.mt_chunk_read
    f.argtypes, f.restype = [P, I, I, I, P], I
    out = {}
    for blocks in (case.batch * case.heads, 6144):
        calls = [(buf.ptr, n, chunk, blocks, sink.ptr) for buf, n in lists]
        per = time_launches(f, calls, steps, warmup)
        nbytes = lists[0][1] * chunk
        out[f'grid_{blocks}'] = dict(us_per_launch=per * 1e6, bytes=nbytes, achieved_gbs=nbytes / per / 1e9,
                                     frac=nbytes / per / 1e9 / PEAK_HBM_GBS)
    n = lists[0][1]
    seq = []
    for _ in lists:
        region = RawDeviceBuffer(n * chunk)
        addrs = RawDeviceBuffer(8 * n)
        addrs.upload(region.ptr + np.arange(n, dtype=np.uint64) * np.uint64(chunk))
        seq.append((region, addrs))
    calls = [(addrs.ptr, n, chunk, 6144, sink.ptr) for _, addrs in seq]
    per = time_launches(f, calls, steps, warmup)
    out['sequential_grid_6144'] = dict(us_per_launch=per * 1e6, bytes=n * chunk,
                                       achieved_gbs=n * chunk / per / 1e9,
                                       frac=n * chunk / per / 1e9 / PEAK_HBM_GBS)
    return out


class no_gc:
    """Python's cyclic garbage collector paused for a timed loop, so that a
    collection does not stall the host between two launches inside the timed
    window (measured: three stalls of 47-58 us within one 200-launch loop)."""

    def __enter__(self):
        self.was = gc.isenabled()
        gc.collect()
        gc.disable()

    def __exit__(self, *exc):
        if self.was:
            gc.enable()


def time_launches(fn, calls, steps, warmup):
    """Mean seconds per launch from HIP events around ``steps`` launches."""
    rt = runtime()
    for i in range(warmup):
        rt.check(fn(*calls[i % len(calls)]))
    rt.synchronize()
    start, end = CudaEvent(), CudaEvent()
    with no_gc():
        start.record()
        for i in range(steps):
            rt.check(fn(*calls[i % len(calls)]))
        end.record()
        rt.synchronize()
    return end.seconds_since(start) / steps


def dropin_config2(case, devs, steps, warmup):
    """Config 2 through ``mt_paged_decode_batch``, the entry the reference's
    decode binds (minitorch/paged_decode.py:65-69): the same rotated pools,
    no host work list, the kernel's own visiting order. Returns the launch
    time and its roofline."""
    from minitorch_amd.dtypes import dtype_code
    fn = paged_ops.paged_library().mt_paged_decode_batch
    fn.argtypes, fn.restype = [P] * 7 + [I] * 10, I
    kw = devs[0].kwargs()
    calls = [(d.out.ptr, d.q.ptr, d.k.ptr, d.v.ptr, d.slab_table.ptr, d.block_table.ptr, d.offsets.ptr,
              kw['b'], kw['h'], kw['d'], kw['page_size'], kw['pages_per_slab'], kw['num_slabs'],
              kw['columns'], kw['layer'], kw['layers'], dtype_code(kw['dtype'])) for d in devs]
    per = time_launches(fn, calls, steps, warmup)
    nbytes = algorithmic_bytes(case)
    achieved = nbytes / per / 1e9
    return dict(entry='mt_paged_decode_batch (reference ABI, include/mt_paged.h)',
                ms_per_step=per * 1e3, tokens_per_sec=case.batch / per,
                roofline={'bound': 'hbm', 'achieved': achieved, 'peak': PEAK_HBM_GBS, 'unit': 'GB/s',
                          'frac': achieved / PEAK_HBM_GBS, 'traffic': None,
                          'algorithmic_bytes_per_launch': nbytes})


def bench_entries(args):
    """The decode entries side by side on config 2, a prologue-bound case of
    its shape (every context 16 tokens, one page), config 4's layer shape and
    config 5 (P = 16): the split entry with a host work list (longest first),
    the split entry in batch order, and the reference-ABI
    mt_paged_decode_batch (its own order); mean launch time from HIP events
    over rotated pools (one pool for config 5, beyond the caches anyway)."""
    from minitorch_amd.workloads import make_decode_case
    from minitorch_amd.runtime import RawDeviceBuffer
    from minitorch_amd.dtypes import dtype_code
    rt = runtime()
    split_fn = paged_ops.paged_library().mt_paged_decode_split
    split_fn.argtypes, split_fn.restype = paged_ops.SPLIT_ARGTYPES, I
    batch_fn = paged_ops.paged_library().mt_paged_decode_batch
    batch_fn.argtypes, batch_fn.restype = [P] * 7 + [I] * 10, I
    from minitorch_amd.e2e import config4_lengths
    from minitorch_amd.workloads import config5_lengths, DeviceRaggedCase
    l4 = config4_lengths(np.random.default_rng([args.seed, 4]), 128)
    l5 = config5_lengths(args.seed, 512)
    one_page = make_decode_case(args.seed, batch=64, heads=12, dim=64, page_size=16, lengths=[16] * 64,
                                pool_pages=8192, pages_per_slab=64, dtype='float16', columns=64)
    # device case lists: host-built pools for configs 2 and the one-page rows,
    # device-filled ones (DeviceRaggedCase) for config 4's layer and config 5
    cases = {
        'config2': lambda: [DevicePagedCase(config2_case(args.seed)) for _ in range(args.pools)],
        'one_page_rows': lambda: [DevicePagedCase(one_page) for _ in range(args.pools)],
        'config4_layer': lambda: [DeviceRaggedCase(args.seed + i, batch=128, heads=16, dim=64, page_size=16,
                                                   lengths=l4, dtype='bfloat16') for i in range(4)],
        'config5_p16': lambda: [DeviceRaggedCase(args.seed, batch=512, heads=25, dim=64, page_size=16,
                                                 lengths=l5, dtype='bfloat16')],
    }
    out = {}
    for name, make in cases.items():
        devs = make()
        case = getattr(devs[0], 'case', devs[0])
        kw = devs[0].kwargs()
        split = paged_ops.split_tokens_for(page_size=case.page_size, columns=case.columns)
        work, items, merges = paged_ops.decode_work_list(case.lengths, case.heads, split, rt.compute_units())
        order = RawDeviceBuffer(4 * len(work))
        order.upload(work)
        base = [(d.out.ptr, d.q.ptr, d.k.ptr, d.v.ptr, d.slab_table.ptr, d.block_table.ptr, d.offsets.ptr,
                 kw['b'], kw['h'], kw['d'], kw['page_size'], kw['pages_per_slab'], kw['num_slabs'],
                 kw['columns'], kw['layer'], kw['layers'], dtype_code(kw['dtype'])) for d in devs]
        ws_bytes = paged_ops.decode_workspace_bytes(b=case.batch, h=case.heads, page_size=case.page_size,
                                                    columns=case.columns, split_tokens=split)
        ws = RawDeviceBuffer(max(ws_bytes, 4))
        tail = (split, args.unroll, args.waves, 0)
        steps = args.steps if case.batch < 512 else min(args.steps, 50)
        times = {
            'split_work_list': time_launches(split_fn, [c + tail + (order.ptr, items, merges, ws.ptr, ws_bytes)
                                                        for c in base], steps, args.warmup),
            'split_batch_order': time_launches(split_fn, [c + tail + (None, 0, 0, ws.ptr, ws_bytes) for c in base],
                                               steps, args.warmup),
            'decode_batch': time_launches(batch_fn, base, steps, args.warmup),
        }
        nbytes = algorithmic_bytes(case)
        out[name] = {k: dict(us_per_launch=t * 1e6, frac=nbytes / t / 1e9 / PEAK_HBM_GBS) for k, t in times.items()}
        del devs, order, ws
    return {'entries': out, 'pools_rotated': args.pools, 'steps': args.steps}


# Compile-time variants of the decode kernel: (name, lanes per token,
# non-temporal K/V loads). The product build is 8 lanes, non-temporal.
DECODE_VARIANTS = (
    ('4_lanes_cached', 4, False),
    ('4_lanes_nt', 4, True),
    ('8_lanes_cached', 8, False),
    ('8_lanes_nt', 8, True),
)
VARIANT_DIR = os.path.join(ROOT, 'build', 'decode_variants')


def build_decode_variants():
    """Builds paged_attention_kernel.so once per DECODE_VARIANTS entry from
    the committed source with its MT_DECODE_GROUP / MT_DECODE_NT_LOADS
    switches, and once with MT_DECODE_TIMELINE (bench_timeline), into
    build/decode_variants/<name>/ (five hipcc processes)."""
    import subprocess
    from minitorch_amd import _build
    src = os.path.join(str(_build.SRC), 'paged_attention_kernel.hip')
    procs = []
    builds = [(name, [f'-DMT_DECODE_GROUP={group}', f'-DMT_DECODE_NT_LOADS={int(nt)}'])
              for name, group, nt in DECODE_VARIANTS]
    builds.append(('timeline', ['-DMT_DECODE_TIMELINE']))  # the product kernel plus per-workgroup stamps
    for name, flags in builds:
        out = os.path.join(VARIANT_DIR, name, 'paged_attention_kernel.so')
        os.makedirs(os.path.dirname(out), exist_ok=True)
        cmd = [_build.hipcc(), *_build.HIPCC_FLAGS, *flags, f'-I{_build.SRC}', src, '-o', out]
        procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    for name, proc in procs:
        _, err = proc.communicate()
        if proc.returncode:
            raise RuntimeError(f'hipcc failed for decode variant {name}:\n{err}')
        print(f'built decode variant {name}', flush=True)


def bench_variants(args):
    """The decode kernel's compile-time variants (DECODE_VARIANTS) x waves per
    workgroup (4, 8) x stream unroll (1, 2, 4), each through its own
    library's mt_paged_decode_split with the host work list: config 2 over
    rotated pools, config 4's layer shape (4 pools) and config 5 at P = 16.
    Mean launch time from HIP events; libraries from build_decode_variants."""
    from minitorch_amd.runtime import RawDeviceBuffer
    from minitorch_amd.dtypes import dtype_code
    from minitorch_amd.e2e import config4_lengths
    from minitorch_amd.workloads import config5_lengths, DeviceRaggedCase
    rt = runtime()
    fns = {}
    for name, _, _ in DECODE_VARIANTS:
        path = os.path.join(VARIANT_DIR, name, 'paged_attention_kernel.so')
        if not os.path.exists(path):
            raise SystemExit(f'{path} is missing: run `python bench.py --build-variants` first')
        fn = ct.CDLL(path).mt_paged_decode_split
        fn.argtypes, fn.restype = paged_ops.SPLIT_ARGTYPES, I
        fns[name] = fn
    l4 = config4_lengths(np.random.default_rng([args.seed, 4]), 128)
    l5 = config5_lengths(args.seed, 512)
    cases = {
        'config2': lambda: [DevicePagedCase(config2_case(args.seed)) for _ in range(args.pools)],
        'config4_layer': lambda: [DeviceRaggedCase(args.seed + i, batch=128, heads=16, dim=64, page_size=16,
                                                   lengths=l4, dtype='bfloat16') for i in range(4)],
        'config5_p16': lambda: [DeviceRaggedCase(args.seed, batch=512, heads=25, dim=64, page_size=16,
                                                 lengths=l5, dtype='bfloat16')],
    }
    out = {}
    for shape, make in cases.items():
        devs = make()
        case = getattr(devs[0], 'case', devs[0])
        kw = devs[0].kwargs()
        split = paged_ops.split_tokens_for(page_size=case.page_size, columns=case.columns)
        work, items, merges = paged_ops.decode_work_list(case.lengths, case.heads, split, rt.compute_units())
        order = RawDeviceBuffer(4 * len(work))
        order.upload(work)
        ws_bytes = paged_ops.decode_workspace_bytes(b=case.batch, h=case.heads, page_size=case.page_size,
                                                    columns=case.columns, split_tokens=split)
        ws = RawDeviceBuffer(max(ws_bytes, 4))
        nbytes = algorithmic_bytes(case)
        steps = args.steps if case.batch < 512 else min(args.steps, 50)
        out[shape] = {}
        for name, fn in fns.items():
            for waves in (4, 8):
                for unroll in (1, 2, 4):
                    calls = [(d.out.ptr, d.q.ptr, d.k.ptr, d.v.ptr, d.slab_table.ptr, d.block_table.ptr,
                              d.offsets.ptr, kw['b'], kw['h'], kw['d'], kw['page_size'], kw['pages_per_slab'],
                              kw['num_slabs'], kw['columns'], kw['layer'], kw['layers'], dtype_code(kw['dtype']),
                              split, unroll, waves, 0, order.ptr, items, merges, ws.ptr, ws_bytes) for d in devs]
                    t = time_launches(fn, calls, steps, args.warmup)
                    out[shape][f'{name}/w{waves}/u{unroll}'] = dict(us_per_launch=round(t * 1e6, 2),
                                                                   frac=round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4))
            print(f'{shape} {name}: ' + ' '.join(f'{k.split("/", 1)[1]} {v["us_per_launch"]:.2f}'
                                                 for k, v in out[shape].items() if k.startswith(name + '/')),
                  file=sys.stderr, flush=True)
        del devs, order, ws
    return {'decode_variants': out, 'pools_rotated': args.pools, 'steps': args.steps}


def bench_timeline(args):
    """Per-workgroup timeline of one cold config-2 launch of the headline path
    (host work list, automatic waves and unroll), from the MT_DECODE_TIMELINE
    build of the decode kernel: each workgroup's start, the arrival of its
    work entry and of its table/query/offset loads, the end of its staging
    barrier, the start of its K/V stream (wave 0) and its end, in µs from the
    launch's first start, with its XCD and compute unit. Summarized as: the
    start spread; prologue steps, stream starts and ends per residency slot
    (workgroups i, i + CUs, i + 2 CUs share a compute unit in a fully resident
    grid); how many workgroups stream over time; the K/V tokens per µs of the
    first slot per XCD; per-CU token loads and their correlation with the
    CU's end time."""
    from minitorch_amd.runtime import RawDeviceBuffer
    from minitorch_amd.dtypes import dtype_code
    path = os.path.join(VARIANT_DIR, 'timeline', 'paged_attention_kernel.so')
    if not os.path.exists(path):
        raise SystemExit(f'{path} is missing: run `python bench.py --build-variants` first')
    lib = ct.CDLL(path)
    fn = lib.mt_paged_decode_split
    fn.argtypes, fn.restype = paged_ops.SPLIT_ARGTYPES, I
    read = lib.mt_decode_timeline
    read.argtypes, read.restype = [ct.POINTER(ct.c_ulonglong), I], I
    rt = runtime()
    if args.config == 4:
        # config 4's layer shape: 128 rows x 16 heads, bf16, more workgroups than one residency round
        from minitorch_amd.e2e import config4_lengths
        from minitorch_amd.workloads import DeviceRaggedCase
        l4 = config4_lengths(np.random.default_rng([args.seed, 4]), 128)
        devs = [DeviceRaggedCase(args.seed + i, batch=128, heads=16, dim=64, page_size=16, lengths=l4,
                                 dtype='bfloat16') for i in range(4)]
        case = devs[0]
    else:
        case = config2_case(args.seed)
        devs = [DevicePagedCase(case) for _ in range(args.pools)]
    kw = devs[0].kwargs()
    split = paged_ops.split_tokens_for(page_size=case.page_size, columns=case.columns)
    cus = rt.compute_units()
    work, items, merges = paged_ops.decode_work_list(case.lengths, case.heads, split, cus)
    order = RawDeviceBuffer(4 * len(work))
    order.upload(work)
    ws_bytes = paged_ops.decode_workspace_bytes(b=case.batch, h=case.heads, page_size=case.page_size,
                                                columns=case.columns, split_tokens=split)
    ws = RawDeviceBuffer(max(ws_bytes, 4))
    calls = [(d.out.ptr, d.q.ptr, d.k.ptr, d.v.ptr, d.slab_table.ptr, d.block_table.ptr, d.offsets.ptr,
              kw['b'], kw['h'], kw['d'], kw['page_size'], kw['pages_per_slab'], kw['num_slabs'],
              kw['columns'], kw['layer'], kw['layers'], dtype_code(kw['dtype']), split, 0, 0, 0,
              order.ptr, items, merges, ws.ptr, ws_bytes) for d in devs]
    for i in range(args.warmup + len(calls)):  # the last launch reads a pool untouched for len(calls) - 1 launches
        rt.check(fn(*calls[i % len(calls)]))
    n = items * case.heads
    fields = 8
    buf = (ct.c_ulonglong * (fields * n))()
    rt.check(read(buf, n))
    rec = np.frombuffer(buf, np.uint64).reshape(n, fields).astype(np.int64)
    t0 = rec[:, 0].min()
    # 100 MHz ticks -> µs from the first start
    start, entry, loads, barrier, stream, end = [(rec[:, j] - t0) / 100.0 for j in range(6)]
    xcc = rec[:, 7] & 0xF
    cu_key = (xcc << 16) | ((rec[:, 6] >> 8) & 0xFF)  # XCD, SE, SH, CU
    rows = work[0:2 * items:2][np.arange(n) // case.heads]
    tokens = case.lengths[rows] - 1  # K/V tokens read from pages (the new one comes from the inputs)
    slot = np.arange(n) // cus
    q = lambda x: [round(float(v), 2) for v in np.quantile(x, [0, 0.5, 1])]
    span = float(end.max())
    grid = np.arange(0, span + 0.25, 0.25)
    streaming = [[round(float(t), 2), int(((stream <= t) & (end > t)).sum())] for t in grid]
    first = slot == 0
    rate = tokens[first] / np.maximum(end[first] - stream[first], 1e-3)
    per_xcd = {int(x): round(float(np.median(rate[xcc[first] == x])), 1) for x in np.unique(xcc[first])}
    keys = np.unique(cu_key)
    cu_tokens = np.array([tokens[cu_key == k].sum() for k in keys])
    cu_end = np.array([end[cu_key == k].max() for k in keys])
    # workgroups dispatched when the launch starts, and those that take a
    # slot freed later (grids of several residency rounds)
    late = start > start.min() + 1.0
    slot_time = float((end - start).sum())
    return {'decode_timeline': {
        'config': 4 if args.config == 4 else 2, 'late_dispatched_workgroups': int(late.sum()),
        'prologue_us_first_dispatch': q(stream[~late] - start[~late]),
        'prologue_us_late_dispatch': q(stream[late] - start[late]) if late.any() else None,
        'stream_us': q(end - stream),
        'prologue_share_of_slot_time': round(float((stream - start).sum()) / slot_time, 3),
        'mean_streaming_workgroups': round(float((end - stream).sum()) / span, 1),
        'workgroups': n, 'compute_units_seen': int(len(keys)), 'span_us': round(span, 2),
        'start_spread_us': round(float(start.max()), 2),
        'prologue_us_by_slot': {int(k): {name: q(v[slot == k]) for name, v in
                                         (('work_entry', entry), ('table_query_offset', loads),
                                          ('staging_barrier', barrier))}
                                for k in np.unique(slot)},
        'stream_start_us_by_slot': {int(k): q(stream[slot == k]) for k in np.unique(slot)},
        'end_us_by_slot': {int(k): q(end[slot == k]) for k in np.unique(slot)},
        'first_slot_tokens_per_us_by_xcd': per_xcd,
        'cu_tokens': q(cu_tokens), 'cu_end_us': q(cu_end),
        'corr_cu_tokens_end': round(float(np.corrcoef(cu_tokens, cu_end)[0, 1]), 3),
        'streaming_workgroups': streaming}}


def bench_config5(args):
    """Config 5: B=512, H=25, D=64, bf16, contexts lognormal(ln 256, 1.2)
    clipped to [1, 8192], page 16 and 32; contexts over 1024 tokens take the
    split-context reduction. The ~1.7 GB of K/V exceeds the Infinity Cache,
    so back-to-back launches read cold data."""
    from minitorch_amd.workloads import DeviceRaggedCase, config5_lengths
    from minitorch_amd.runtime import RawDeviceBuffer
    from minitorch_amd.dtypes import dtype_code
    rt = runtime()
    lengths = config5_lengths(args.seed, 512)
    lines = {}
    fn = paged_ops.paged_library().mt_paged_decode_split
    fn.argtypes, fn.restype = paged_ops.SPLIT_ARGTYPES, I
    for page_size in (16, 32):
        case = DeviceRaggedCase(args.seed, batch=512, heads=25, dim=64, page_size=page_size,
                                lengths=lengths, dtype='bfloat16')
        kw = case.kwargs()
        split = paged_ops.split_tokens_for(page_size=page_size, columns=case.columns, requested=args.split)
        ws_bytes = paged_ops.decode_workspace_bytes(b=512, h=25, page_size=page_size,
                                                    columns=case.columns, split_tokens=split)
        ws = RawDeviceBuffer(max(ws_bytes, 4))
        work, items, merges = paged_ops.decode_work_list(case.lengths, 25, split, rt.compute_units())
        order = RawDeviceBuffer(4 * len(work))
        order.upload(work)
        work_args = (None, 0, 0) if args.natural_order else (order.ptr, items, merges)
        call = (case.out.ptr, case.q.ptr, case.k.ptr, case.v.ptr, case.slab_table.ptr,
                case.block_table.ptr, case.offsets.ptr, kw['b'], kw['h'], kw['d'], kw['page_size'],
                kw['pages_per_slab'], kw['num_slabs'], kw['columns'], kw['layer'], kw['layers'],
                dtype_code(kw["dtype"]), split, args.unroll, args.waves, 0, *work_args, ws.ptr, ws_bytes)
        per = time_launches(fn, [call], min(args.steps, 50), min(args.warmup, 5))
        # the reference-ABI entry on the same case: no work list, its own
        # workspace and visiting order
        batch_fn = paged_ops.paged_library().mt_paged_decode_batch
        batch_fn.argtypes, batch_fn.restype = [P] * 7 + [I] * 10, I
        per_batch = time_launches(batch_fn, [call[:17]], min(args.steps, 50), min(args.warmup, 5))
        s = 2
        L = case.lengths
        nbytes = (512 * 25 * 64 * 2 * (s + s) + int((2 * L * 25 * 64 * s).sum()) + 512 * 25 * 64 * (s + s)
                  + int((4 * ((L + page_size - 1) // page_size)).sum()) + 4 * 512)
        lines[page_size] = dict(ms_per_step=per * 1e3, tokens_per_sec=512 / per,
                                achieved_gbs=nbytes / per / 1e9, frac=nbytes / per / 1e9 / PEAK_HBM_GBS,
                                algorithmic_bytes=nbytes, columns=case.columns,
                                rows_over_1024=int((L > 1024).sum()), max_context=int(L.max()),
                                dropin=dict(entry='mt_paged_decode_batch', ms_per_step=per_batch * 1e3,
                                            achieved_gbs=nbytes / per_batch / 1e9,
                                            frac=nbytes / per_batch / 1e9 / PEAK_HBM_GBS))
        if page_size == 16 and not args.no_cpu_baseline:
            lines['cpu_baseline'] = ragged_cpu_baseline(case, args.cpu_seconds)
        del case, ws, order
    main16 = lines[16]
    return {
        'metric': METRIC, 'value': main16['tokens_per_sec'], 'unit': 'tokens/s', 'n_gpus': 1,
        'steps': min(args.steps, 50), 'warmup': min(args.warmup, 5), 'ms_per_step': main16['ms_per_step'],
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16',
        'data': 'synthetic (hash-filled K/V)',
        'config': {'workload': 'config 5: ragged op-level paged decode, B=512, H=25, D=64, bf16, '
                               'L~lognormal(ln 256, 1.2) clipped [1, 8192], split reduction for L>1024',
                   'sum_context_tokens': int(lengths.sum()), 'split_tokens': split},
        'roofline': {'bound': 'hbm', 'achieved': main16['achieved_gbs'], 'peak': PEAK_HBM_GBS,
                     'unit': 'GB/s', 'frac': main16['frac'], 'traffic': None,
                     'algorithmic_bytes_per_launch': main16['algorithmic_bytes']},
        'page_size_16': lines[16], 'page_size_32': lines[32],
        'cpu_baseline': lines.get('cpu_baseline'),
    }


def prefill_flops(n, heads, dim):
    """Causal attention flops of one n-token prompt: q.k and p.v over the
    n(n+1)/2 attended (query, key) pairs, 2 flops per multiply-add."""
    return 2.0 * heads * dim * n * (n + 1)


def bench_prefill_shape(heads, dtype, lengths, steps, warmup, seed):
    """Mean time of mt_paged_attention over prompts of the given lengths (one
    request per call, nq = nk = n, offset 0), the pages of all prompts in one
    shuffled pool."""
    from minitorch_amd.workloads import make_decode_case
    from minitorch_amd.runtime import DeviceTensor
    from minitorch_amd.dtypes import dtype_code
    dim, page = 64, 16
    lengths = np.asarray(lengths, np.int64)
    pages = int(((lengths + page - 1) // page).sum())
    case = make_decode_case(seed, batch=len(lengths), heads=heads, dim=dim, page_size=page,
                            lengths=lengths, pool_pages=-(-pages // 16) * 16, pages_per_slab=16,
                            dtype=dtype)
    dev = DevicePagedCase(case)
    nmax = int(lengths.max())
    q = DeviceTensor((1, heads, nmax, dim), dtype)
    rt = runtime()
    from minitorch_amd.workloads import _normal
    rt.h2d(q.ptr, _normal(np.random.default_rng([seed, 6]), (1, heads, nmax, dim), dtype))
    out = DeviceTensor((1, heads, nmax, dim), dtype)
    fn = paged_ops.paged_library().mt_paged_attention
    fn.argtypes, fn.restype = [P] * 4 + [I] * 13, I
    calls = [(out.ptr, q.ptr, dev.slab_table.ptr, dev.block_table.ptr + 4 * i * case.columns, 1, heads,
              int(n), int(n), dim, page, case.pages_per_slab, case.num_slabs, case.columns, 0, 1, 0,
              dtype_code(dtype)) for i, n in enumerate(lengths)]
    per_round = time_launches(fn, calls, steps * len(calls), warmup * len(calls)) * len(calls)
    flops = sum(prefill_flops(int(n), heads, dim) for n in lengths)
    return dict(prompts=len(lengths), mean_prompt=float(lengths.mean()), max_prompt=nmax,
                us_per_prefill=per_round / len(calls) * 1e6, tflops=flops / per_round / 1e12,
                frac=flops / per_round / 1e12 / PEAK_MFMA_TFLOPS)


def bench_prefill_ragged(heads, dtype, lengths, steps, warmup, seed, per_call=16):
    """Mean time per prompt of mt_paged_prefill_ragged (append + causal
    attention) over the same prompts, ``per_call`` prompts per call
    (token-major rows of one fused QKV buffer, as the batched prefill loop
    passes them)."""
    from minitorch_amd.workloads import make_decode_case, _normal
    from minitorch_amd.runtime import DeviceTensor
    from minitorch_amd.dtypes import dtype_code
    dim, page = 64, 16
    lengths = np.asarray(lengths, np.int64)
    pages = int(((lengths + page - 1) // page).sum())
    case = make_decode_case(seed, batch=len(lengths), heads=heads, dim=dim, page_size=page,
                            lengths=lengths, pool_pages=-(-pages // 16) * 16, pages_per_slab=16,
                            dtype=dtype)
    dev = DevicePagedCase(case)
    hd, total = heads * dim, int(lengths.sum())
    qkv = DeviceTensor((total, 3 * hd), dtype)
    rt = runtime()
    rt.h2d(qkv.ptr, _normal(np.random.default_rng([seed, 7]), (total, 3 * hd), dtype))
    out = DeviceTensor((total, hd), dtype)
    fn = paged_ops.paged_library().mt_paged_prefill_ragged
    fn.argtypes, fn.restype = [P] * 8 + [I] * 12, I
    calls, row = [], 0
    for c0 in range(0, len(lengths), per_call):
        sel = range(c0, min(c0 + per_call, len(lengths)))
        n = [int(lengths[i]) for i in sel]
        tables = (P * len(n))(*[dev.block_table.ptr + 4 * i * case.columns for i in sel])
        item = 2
        calls.append((out.ptr + row * hd * item, qkv.ptr + row * 3 * hd * item,
                      qkv.ptr + (row * 3 * hd + hd) * item, qkv.ptr + (row * 3 * hd + 2 * hd) * item,
                      dev.slab_table.ptr, tables, (I * len(n))(*n), (I * len(n))(*([0] * len(n))), len(n), heads,
                      dim, page, case.pages_per_slab, case.num_slabs, case.columns, 0, 1, dtype_code(dtype),
                      3 * hd, hd))
        row += sum(n)
    per_round = time_launches(fn, calls, steps * len(calls), warmup * len(calls)) * len(calls)
    flops = sum(prefill_flops(int(n), heads, dim) for n in lengths)
    return dict(prompts=len(lengths), prompts_per_call=per_call, us_per_prompt=per_round / len(lengths) * 1e6,
                tflops=flops / per_round / 1e12, frac=flops / per_round / 1e12 / PEAK_MFMA_TFLOPS)


def prefill_cpu_baseline(heads, dtype, lengths, seed, seconds):
    """The C oracle's causal paged attention (oracle_paged_attention) over the
    same prompts and pages as :func:`bench_prefill_shape`, one prompt per call,
    the prompts spread over a pool of host threads (one OpenMP thread per
    call), repeated until ``seconds`` have passed."""
    from concurrent.futures import ThreadPoolExecutor
    from minitorch_amd.workloads import make_decode_case, _normal
    try:
        from oracle import c_oracle
        lib = c_oracle.library()
    except Exception as error:  # the oracle library is optional on the GPU box
        return dict(value=None, unit='TFLOP/s', cores=None, kind='port', sample=f'unavailable: {error}')
    dim, page = 64, 16
    lengths = np.asarray(lengths, np.int64)
    pages = int(((lengths + page - 1) // page).sum())
    case = make_decode_case(seed, batch=len(lengths), heads=heads, dim=dim, page_size=page,
                            lengths=lengths, pool_pages=-(-pages // 16) * 16, pages_per_slab=16,
                            dtype=dtype)
    nmax = int(lengths.max())
    q = np.ascontiguousarray(_normal(np.random.default_rng([seed, 6]), (1, heads, nmax, dim), dtype))
    image = np.ascontiguousarray(case.image)
    slabs = np.array([image.ctypes.data + s * case.slab_bytes for s in range(case.num_slabs)], np.uint64)
    table = np.ascontiguousarray(case.table, np.int32)
    code = c_oracle.CODES[dtype]

    def one(i):
        n = int(lengths[i])
        qi = np.ascontiguousarray(q[:, :, :n])
        out = np.empty_like(qi)
        status = lib.oracle_paged_attention(out.ctypes.data, qi.ctypes.data, slabs.ctypes.data,
                                            table.ctypes.data + 4 * i * case.columns, 1, heads, n, n, dim,
                                            page, case.pages_per_slab, case.num_slabs, case.columns, 0, 1, 0,
                                            code, 1)
        if status:
            raise RuntimeError(f'oracle_paged_attention returned {status}')

    threads = min(os.cpu_count() or 1, 16)
    flops = sum(prefill_flops(int(n), heads, dim) for n in lengths)
    with ThreadPoolExecutor(threads) as pool:
        rounds, t0 = 0, time.perf_counter()
        while True:
            list(pool.map(one, range(len(lengths))))
            rounds += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= seconds:
                break
    return dict(value=flops * rounds / elapsed / 1e12, unit='TFLOP/s', cores=threads, kind='port',
                sample=f'{rounds} passes over the {len(lengths)} prompts in {elapsed:.1f} s, fp32 arithmetic '
                       f'on {dtype} pages, one prompt per call, {threads} host threads')


def bench_prefill(args):
    """Causal paged prefill attention (the matrix-core kernel behind
    mt_paged_attention) on the prompt shapes of configs 3 and 4: config 3's
    first 64 prompts (U{32..512}, 12 heads, fp16) and 64 config-4 contexts
    (lognormal median 256, clipped [16, 1024], 16 heads, bf16), one request per
    call as the batcher admits them, plus single 512- and 1024-token prompts;
    and the same prompts through mt_paged_prefill_ragged, 16 per call (append
    included), as the batched prefill loop issues them."""
    from minitorch_amd.e2e import config3_trace, config4_lengths
    steps, warmup = max(1, args.steps // 20), max(1, args.warmup // 10)
    c3 = [len(p) for _, _, p, _ in config3_trace(args.seed)[:64]]
    c4 = config4_lengths(np.random.default_rng([args.seed, 4]), 64)
    r3 = bench_prefill_shape(12, 'float16', c3, steps, warmup, args.seed)
    r4 = bench_prefill_shape(16, 'bfloat16', c4, steps, warmup, args.seed)
    r512 = bench_prefill_shape(12, 'float16', [512], steps * 20, warmup * 10, args.seed)
    r1024 = bench_prefill_shape(16, 'bfloat16', [1024], steps * 20, warmup * 10, args.seed)
    rr3 = bench_prefill_ragged(12, 'float16', c3, steps, warmup, args.seed)
    rr4 = bench_prefill_ragged(16, 'bfloat16', c4, steps, warmup, args.seed)
    return {'metric': 'causal paged prefill attention TFLOP/s (1 GPU)', 'value': r3['tflops'],
            'unit': 'TFLOP/s', 'n_gpus': 1, 'steps': steps, 'warmup': warmup,
            'ms_per_step': r3['us_per_prefill'] * r3['prompts'] / 1e3, 'higher_is_better': True,
            'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f16', 'data': 'synthetic',
            'config': {'workload': 'config-3 prompt shapes: 64 prompts U{32..512}, 12 heads, D 64, page 16, '
                                   'fp16, one request per mt_paged_attention call (a step = the 64 calls)'},
            'roofline': {'bound': 'mfma', 'achieved': r3['tflops'], 'peak': PEAK_MFMA_TFLOPS,
                         'unit': 'TFLOP/s', 'frac': r3['frac'], 'traffic': None},
            'config3_prompts_fp16': r3, 'config4_contexts_bf16': r4, 'prompt512_h12_fp16': r512,
            'prompt1024_h16_bf16': r1024,
            'config3_prompts_fp16_ragged16': rr3, 'config4_contexts_bf16_ragged16': rr4,
            'cpu_baseline': None if args.no_cpu_baseline else prefill_cpu_baseline(
                12, 'float16', c3, args.seed, args.cpu_seconds)}


def e2e_cpu_baseline(model, lengths, seconds, seed):
    """Decode steps of the same architecture on the host: the oracle's
    KV-cached batched decode (numpy fp32, BLAS threads for the projections)
    over caches of the given context lengths (capped 16 below the position
    limit, so that steps can follow) holding zero K/V (a step's cost does not
    depend on their values), median step time over ``seconds`` (at least 10
    steps)."""
    from oracle import gpt2_oracle as go
    rng = np.random.default_rng([seed, 7])
    state = go._cast(model.state, np.float32)
    hd = model.n_embd // model.n_head
    lengths = [min(int(n), model.n_positions - 16) for n in lengths]
    room = model.n_positions - max(lengths)
    caches = [{'length': n, 'k': [np.zeros((model.n_head, n + room, hd), np.float32) for _ in range(model.n_layer)],
               'v': [np.zeros((model.n_head, n + room, hd), np.float32) for _ in range(model.n_layer)]}
              for n in lengths]
    ids = rng.integers(0, model.n_vocab, len(lengths))
    start = [c['length'] for c in caches]

    def step():
        nonlocal ids
        if caches[0]['length'] - start[0] >= room - 1:  # rewind: same work per step
            for c, n in zip(caches, start):
                c['length'] = n
        ids = go.decode_step(state, caches, ids, n_head=model.n_head, n_layer=model.n_layer).argmax(axis=1)

    many = timed_steps(step, seconds)
    try:
        from threadpoolctl import threadpool_info
        threads = max((p.get('num_threads', 1) for p in threadpool_info()), default=None)
    except Exception:
        threads = None
    return dict(value=len(lengths) / float(np.median(many)), unit='tokens/s', cores=threads, kind='port',
                sample=f'median of {len(many)} decode steps ({many.sum():.1f} s) of B={len(lengths)} rows, contexts '
                       f'{min(lengths)}..{max(lengths)} (mean {np.mean(lengths):.0f}), numpy fp32 KV-cached '
                       f'decode (oracle/gpt2_oracle.py), zero K/V',
                host=dict(nproc=os.cpu_count(), cpu_model=host_cpu_model()))


def bench_projections(args):
    """Decode projections of DistilGPT-2 (fp16) and GPT-2-medium (bf16) at a
    few batch sizes: the matrix-core projection kernel (mt_decode_projection,
    with the split the decoder loop chooses for the out- and proj-projections)
    on row-major operands and on fragment-tiled ones (the weights, and the
    activations of qkv, fc and proj; fc also writes its output tiled, as in the
    decoder loop) against hipBLASLt
    (mt_gemm_ex with bias), each over enough distinct copies
    of the weights (>= 512 MiB) that every launch reads them from HBM, the
    launches of one kind captured in a HIP graph and replayed; microseconds
    per launch."""
    from minitorch_amd.model import model_library, DecoderLM
    from minitorch_amd.runtime import DeviceTensor, call
    from minitorch_amd.dtypes import dtype_code
    rt = runtime()
    lib = model_library()
    proj_args = [P, P, P, P, I, I, I, I, I, I, I]
    gemm_args = [P, P, P, P, P, I, I, I, I, I, I]
    blas = DecoderLM(n_vocab=16, n_embd=16, n_head=1, n_layer=1, n_positions=4).blas()

    def filled(shape, seed, dtype):
        t = DeviceTensor(shape, dtype)
        rt.check(rt.lib.mt_fill_random(t.ptr, int(np.prod(shape)), seed, dtype_code(dtype)))
        return t

    def waves_ok(rng, q):
        smax = 2 if q >= 8 else 4
        return any(rng % (32 * w) == 0 and rng // (32 * w) <= smax for w in range(16, 0, -1))

    def splits(m, n, k):
        # the decoder loop's choice (proj_tiles and projection_splits in csrc/model_kernels.hip)
        if m <= 32:
            mt, nt = (1 if m <= 16 else 2), 1
        elif n % 32 == 0:
            mt, nt = (2 if m <= 64 else 4), 2
        else:
            mt, nt = (4 if m <= 64 else 8), 1
        tiles, s = n // (16 * nt) * -(-m // (16 * mt)), 1
        while s < 8 and not (k % s == 0 and waves_ok(k // s, mt * nt)):
            s *= 2
        while s < 8 and tiles * s < rt.compute_units() and k % (2 * s) == 0 and waves_ok(k // (2 * s), mt * nt):
            s *= 2
        return s

    def graph_time(launch, reps=5):
        launch()
        rt.synchronize()
        rt.check(rt.lib.mt_graph_begin())
        launch()
        ex = ct.c_void_p()
        rt.check(rt.lib.mt_graph_end(ct.byref(ex)))
        rt.check(rt.lib.mt_graph_launch(ex))
        rt.synchronize()
        e0, e1 = CudaEvent(), CudaEvent()
        e0.record()
        for _ in range(reps):
            rt.check(rt.lib.mt_graph_launch(ex))
        e1.record()
        e1.synchronize()
        rt.check(rt.lib.mt_graph_destroy(ex))
        return e1.seconds_since(e0) / reps

    rows = []
    for name, d, dtype, ms in (('distilgpt2', 768, 'float16', (2, 16, 64, 128)),
                               ('gpt2-medium', 1024, 'bfloat16', (2, 16, 32, 64, 128, 256))):
        code = dtype_code(dtype)
        for m in ms:
            x = filled((m, 4 * d), 1, dtype)
            xt = filled((-(-m // 16) * 16, 4 * d), 3, dtype)  # the tiled layout's padded rows
            bias = filled((4 * d,), 2, dtype)
            out = DeviceTensor((8, m, 4 * d), 'float32')
            for kind, n, k, epi in (('qkv', 3 * d, d, 0), ('out', d, d, 2), ('fc', 4 * d, d, 1),
                                    ('proj', d, 4 * d, 2)):
                sp = splits(m, n, k) if epi == 2 else 1
                copies = max(8, -(-(512 << 20) // (n * k * 2)))
                ws = [filled((n, k), 100 + i, dtype) for i in range(copies)]

                def own(layout=0):
                    for w in ws:
                        call(lib, 'mt_decode_projection', proj_args, out.ptr, xt.ptr if layout else x.ptr, w.ptr,
                             0 if epi == 2 else bias.ptr, m, n, k, sp, epi, code, layout)

                def hipblaslt():
                    for w in ws:
                        call(lib, 'mt_gemm_ex', gemm_args, blas.handle, out.ptr, x.ptr, w.ptr, bias.ptr, m, n, k, 1,
                             code, code)
                t_own, t_blas = graph_time(own) / copies, graph_time(hipblaslt) / copies
                rows.append(dict(model=name, rows=m, projection=kind, n=n, k=k, splits=sp,
                                 epilogue=('bias', 'bias+gelu', 'split partials')[epi],
                                 own_us=round(t_own * 1e6, 2), hipblaslt_us=round(t_blas * 1e6, 2)))
                # tiled weights, and tiled activations except for out (attention's row-major output)
                layout = 4 | (0 if kind == 'out' else 3 if kind == 'fc' else 1)
                rows[-1]['own_tiled_us'] = round(graph_time(lambda: own(layout)) / copies * 1e6, 2)
                print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
                del ws
    return dict(metric='decode projection time (us per launch, cold weights)', projections=rows)


def e2e_config3(args, loops=('sync', 'sync-free')):
    """Config 3 end to end: the 256-request DistilGPT-2 trace (fp16) replayed by
    wall clock through the batcher. Reports decode tokens/s by the reference's
    formula (generated tokens / (end - start), arrival gaps included,
    project/benchmark_continuous_batching.py:122) and as busy-step tokens/s
    (decode tokens / time of the steps that ran), per loop."""
    from minitorch_amd import model as model_mod, e2e
    model = model_mod.distilgpt2(seed=args.seed)
    trace = e2e.config3_trace(args.seed)
    warm = e2e.config3_trace(args.seed + 1, requests=8, rate=1000.0)
    r = {}
    if 'sync' in loops:
        e2e.run_config3(model, warm, precision='fp16', report_every=0)
        r = e2e.run_config3(model, trace, precision='fp16')
    if 'sync-free' in loops:
        # the same trace through the sync-free loop (device-side token feedback)
        e2e.run_config3(model, warm, precision='fp16', token_feedback=True, report_every=0)
        r['sync_free'] = e2e.run_config3(model, trace, precision='fp16', token_feedback=True)
        # and with each decode step replayed from a HIP graph (one per batch size)
        e2e.run_config3(model, warm, precision='fp16', token_feedback=True, graph=True, report_every=0)
        r['graph'] = e2e.run_config3(model, trace, precision='fp16', token_feedback=True, graph=True)
        # graph replay of decode-only steps, and steps that admit run decode
        # and prefill as one layer loop
        r['merged'] = e2e.run_config3(model, trace, precision='fp16', token_feedback=True, graph=True,
                                      merge_prefill=True)
    if not args.no_cpu_baseline:
        # the trace's mean decode batch, mid-generation contexts of its first requests
        batch = max(1, int(round((r.get('sync_free') or r).get('mean_decode_batch_size', 2))))
        r['cpu_baseline'] = e2e_cpu_baseline(model, [len(p) + 64 for _, _, p, _ in trace[:batch]],
                                             args.cpu_seconds, args.seed)
    r['workload'] = ('config 3: continuous batching, random-init DistilGPT-2 (6 layers, d 768, 12 heads, vocab '
                     '50257), fp16, 256 Poisson requests at 32 req/s, prompts U[32,512], outputs geometric mean '
                     '128, greedy, EOS off, 16384 pages of 16 tokens, FIFO, max_batch_size 256')
    return r


def e2e_config4(args, loops=('sync', 'sync-free')):
    """Config 4 end to end: 128 concurrent GPT-2-medium (bf16) requests, 5 %
    replaced per step. Reports decode tokens/s and ms per decode step (whole
    24-layer model step with the tied head, tokens to the host) and the whole
    loop's rate including the replacement prefills, per loop; the merged loop
    (decode and replacement prefills of a step in one layer loop) reports the
    whole loop's rate only."""
    from minitorch_amd import model as model_mod, e2e
    distil = args.model == 'distilgpt2'
    model = model_mod.distilgpt2(seed=args.seed) if distil else model_mod.gpt2_medium(seed=args.seed)
    kw = dict(seed=args.seed, steps=max(10, min(args.steps, 40)), warmup=max(2, min(args.warmup, 5)),
              replace_rate=args.replace_rate, batch_prefills=not args.prefill_each, concurrent=args.concurrent,
              precision='fp16' if distil else 'bf16')
    r = e2e.run_config4(model, **kw) if 'sync' in loops else {}
    if 'sync-free' in loops:
        r['sync_free'] = e2e.run_config4(model, **kw, token_feedback=True)
        # the sync-free loop with each decode step replayed from a HIP graph
        r['graph'] = e2e.run_config4(model, **kw, token_feedback=True, graph=True)
    if 'sync-free' in loops or 'merged' in loops:
        # the sync-free loop with each step's decode and replacement prefills
        # in one layer loop
        r['merged'] = e2e.run_config4(model, **kw, token_feedback=True, merge_prefill=True)
    if not args.no_cpu_baseline:
        r['cpu_baseline'] = e2e_cpu_baseline(
            model, e2e.config4_lengths(np.random.default_rng([args.seed, 4]), args.concurrent),
            args.cpu_seconds, args.seed)
    arch = ('DistilGPT-2 (6 layers, d 768, 12 heads), fp16' if distil
            else 'GPT-2-medium (24 layers, d 1024, 16 heads), bf16')
    r['workload'] = (f'config 4: steady state of {args.concurrent} requests, random-init {arch}, contexts '
                     'lognormal(median 256, sigma 1.2) clipped [16,1024], page 16, '
                     f'{args.replace_rate:.0%} replaced per step')
    return r


def config1_times(args):
    """Config 1 (4 requests, L = {7, 33, 64, 120}, 12 heads, fp32): one
    mt_paged_decode_batch launch on the GPU (HIP events, mean of many) and the
    C restatement's decode step on the host (median, 1 and up to 16 threads)."""
    from minitorch_amd.workloads import config1_case
    case = config1_case(args.seed)
    dev = DevicePagedCase(case)
    fn = paged_ops.paged_library().mt_paged_decode_batch
    fn.argtypes, fn.restype = [P] * 7 + [I] * 10, I
    from minitorch_amd.dtypes import dtype_code
    kw = dev.kwargs()
    call = (dev.out.ptr, dev.q.ptr, dev.k.ptr, dev.v.ptr, dev.slab_table.ptr, dev.block_table.ptr,
            dev.offsets.ptr, kw['b'], kw['h'], kw['d'], kw['page_size'], kw['pages_per_slab'], kw['num_slabs'],
            kw['columns'], kw['layer'], kw['layers'], dtype_code(kw['dtype']))
    per = time_launches(fn, [call], 200, 20)
    out = dict(workload='config 1: B=4, L={7,33,64,120}, H=12, D=64, P=16, fp32, 64-page pool',
               gpu_us_per_launch=per * 1e6)
    if args.no_cpu_baseline:
        return out
    try:
        from oracle import c_oracle
        lib = c_oracle.library()
    except Exception as error:  # the oracle library is optional on the GPU box
        out['cpu_baseline'] = dict(value=None, sample=f'unavailable: {error}')
        return out
    host = c_oracle.HostCase(case)
    threads = min(os.cpu_count() or 1, 16)
    seconds = min(2.0, args.cpu_seconds)
    many = timed_steps(lambda: host.run(lib, threads), seconds)
    one = timed_steps(lambda: host.run(lib, 1), seconds)
    out['cpu_baseline'] = dict(value=float(np.median(many)) * 1e6, unit='us per step', cores=threads, kind='port',
                               sample=f'median of {len(many)} config-1 decode steps (append + attention), fp32, '
                                      f'C restatement, OpenMP over (request, head)',
                               single_core=dict(value=float(np.median(one)) * 1e6, unit='us per step', cores=1,
                                                steps=len(one)))
    return out


def bench_e2e(args):
    if args.config == 3:
        if args.loop == 'merged':
            raise SystemExit('--loop merged applies to config 4')
        loops = ('sync', 'sync-free') if args.loop == 'both' else (args.loop,)
        r = e2e_config3(args, loops)
        value, dtype = (r.get('busy_decode_tokens_per_sec') or r.get('sync_free', {}).get('busy_step_tokens_per_sec')), 'f16'
    else:
        loops = ('sync', 'sync-free') if args.loop == 'both' else (args.loop,)
        r = e2e_config4(args, loops)
        value = (r.get('decode_tokens_per_sec') or r.get('sync_free', {}).get('loop_tokens_per_sec') or
                 r.get('merged', {}).get('loop_tokens_per_sec'))
        dtype = 'f16' if args.model == 'distilgpt2' else 'bf16'
    return {'metric': 'decode tokens/s (1 GPU), end to end', 'value': value, 'unit': 'tokens/s',
            'n_gpus': 1, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
            'dtype': dtype, 'data': 'synthetic (random-init weights, random token ids)',
            'config': {'workload': r.pop('workload')}, 'cpu_baseline': r.pop('cpu_baseline', None),
            'measurements': r}


# The reference's published DistilGPT-2 figures (pretrained weights, fp32, one
# RTX 4060 Laptop GPU; README.md:267-281, docs/images/01_inference_modes.png,
# docs/images/02_continuous_batching.png): context beside this build's
# numbers, not a target.
REFERENCE_PUBLISHED = {
    'hardware': 'RTX 4060 Laptop GPU 8 GB, fp32, pretrained DistilGPT-2',
    'trace': {'serial': {'output_tokens_per_sec': 87.60, 'ttft_p50_ms': 289.16, 'ttft_p95_ms': 483.22,
                         'kv_reserved_peak_mib': 20.25},
              'continuous': {'output_tokens_per_sec': 184.92, 'ttft_p50_ms': 40.47, 'ttft_p95_ms': 89.31,
                             'max_decode_batch_size': 4, 'mean_decode_batch_size': 2.84,
                             'kv_reserved_peak_mib': 36.00},
              'continuous_vs_serial': 2.11},
    'inference_modes_paged': {'32': {'decode_tokens_per_sec': 84.77, 'output_tokens_per_sec': 83.87,
                                     'median_ttft_ms': 13.47},
                              '128': {'decode_tokens_per_sec': 86.41, 'output_tokens_per_sec': 84.66,
                                      'median_ttft_ms': 15.76},
                              '256': {'decode_tokens_per_sec': 87.62, 'output_tokens_per_sec': 84.46,
                                      'median_ttft_ms': 18.13},
                              '512': {'decode_tokens_per_sec': 92.30, 'output_tokens_per_sec': 78.86,
                                      'median_ttft_ms': 40.40}},
}


def reference_scenarios(args):
    """The reference's two published scenarios on random-init DistilGPT-2 in
    fp32 (minitorch_amd.e2e.run_reference_scenarios): the serial vs
    continuous trace and batch-1 paged inference at 32-512-token prompts, 1
    warmup and 3 measured runs each, beside the reference's own figures."""
    from minitorch_amd import e2e, model as model_mod
    model = model_mod.distilgpt2(seed=args.seed)
    r = e2e.run_reference_scenarios(model, seed=args.seed)
    r['workload'] = ('DistilGPT-2 architecture, random-init weights, synthetic prompt IDs of the reference '
                     'lengths, fp32, KV budget 256 MiB, pages of 16 tokens, 4 pages per slab')
    r['reference_published'] = REFERENCE_PUBLISHED
    return r


def e2e_summary(r3, r4):
    """The end-to-end figures of configs 3 and 4 for the default line."""
    out = {}
    if r3 is not None:
        sf, gr, mg = r3.get('sync_free', {}), r3.get('graph', {}), r3.get('merged', {})
        out['config3'] = dict(
            workload=r3['workload'],
            decode_tokens_per_sec_reference_formula=r3.get('output_tokens_per_sec'),
            busy_step_decode_tokens_per_sec=r3.get('busy_step_tokens_per_sec'),
            busy_decode_tokens_per_sec=r3.get('busy_decode_tokens_per_sec'),
            sync_free=dict(decode_tokens_per_sec_reference_formula=sf.get('output_tokens_per_sec'),
                           busy_step_decode_tokens_per_sec=sf.get('busy_step_tokens_per_sec'),
                           ttft_p50_ms=sf.get('ttft_p50_ms')) if sf else None,
            graph=dict(decode_tokens_per_sec_reference_formula=gr.get('output_tokens_per_sec'),
                       busy_step_decode_tokens_per_sec=gr.get('busy_step_tokens_per_sec'),
                       ttft_p50_ms=gr.get('ttft_p50_ms'), completed=gr.get('completed')) if gr else None,
            merged=dict(decode_tokens_per_sec_reference_formula=mg.get('output_tokens_per_sec'),
                        busy_step_decode_tokens_per_sec=mg.get('busy_step_tokens_per_sec'),
                        ttft_p50_ms=mg.get('ttft_p50_ms'), completed=mg.get('completed'),
                        kv_pool_used_pages_after=mg.get('kv_pool_used_pages_after')) if mg else None,
            elapsed_seconds=r3.get('elapsed_seconds'), generated_tokens=r3.get('generated_tokens'),
            completed=r3.get('completed'), mean_decode_batch_size=r3.get('mean_decode_batch_size'),
            ttft_p50_ms=r3.get('ttft_p50_ms'), ttft_p95_ms=r3.get('ttft_p95_ms'),
            kv_pool_used_pages_after=r3.get('kv_pool_used_pages_after'),
            cpu_baseline=r3.get('cpu_baseline'))
    if r4 is not None:
        sf, gr, mg = r4.get('sync_free', {}), r4.get('graph', {}), r4.get('merged', {})
        out['config4'] = dict(
            workload=r4['workload'],
            decode_tokens_per_sec=r4.get('decode_tokens_per_sec'), ms_per_decode_step=r4.get('ms_per_step'),
            loop_tokens_per_sec=r4.get('loop_tokens_per_sec'), loop_ms_per_step=r4.get('loop_ms_per_step'),
            sync_free=dict(loop_tokens_per_sec=sf.get('loop_tokens_per_sec'),
                           loop_ms_per_step=sf.get('loop_ms_per_step'),
                           decode_ms_per_step=sf.get('ms_per_step')) if sf else None,
            graph=dict(decode_tokens_per_sec=gr.get('decode_tokens_per_sec'),
                       decode_ms_per_step=gr.get('ms_per_step'),
                       loop_tokens_per_sec=gr.get('loop_tokens_per_sec'),
                       loop_ms_per_step=gr.get('loop_ms_per_step')) if gr else None,
            merged=dict(loop_tokens_per_sec=mg.get('loop_tokens_per_sec'),
                        loop_ms_per_step=mg.get('loop_ms_per_step'),
                        replaced_requests=mg.get('replaced_requests')) if mg else None,
            steps=r4.get('steps'), mean_context_tokens=r4.get('mean_context_tokens'),
            replaced_requests=r4.get('replaced_requests'), page_reuses=r4.get('page_reuses'),
            cpu_baseline=r4.get('cpu_baseline'))
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--pools', type=int, default=6)
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--split', type=int, default=0, help='split length in tokens (0 = automatic)')
    ap.add_argument('--unroll', type=int, default=0)
    ap.add_argument('--waves', type=int, default=0, help='waves per decode workgroup (2, 4 or 8; 0 = default)')
    ap.add_argument('--natural-order', action='store_true',
                    help='no work list: schedule every (split, row) in batch order')
    ap.add_argument('--cpu-seconds', type=float, default=10.0)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--calibrate-copy', type=int, default=0, metavar='MB',
                    help='only run device-to-device copies of MB MiB (counter calibration) and exit')
    ap.add_argument('--no-ceiling', action='store_true',
                    help='config 2: skip timing the plain kernel that reads exactly the K/V pages of the '
                         'step (2 KiB page-head chunks, no math), reported as pattern_ceiling')
    ap.add_argument('--config', type=int, default=2, choices=(2, 3, 4, 5),
                    help='2: op-level decode (default, the headline line); 5: ragged op-level '
                         'decode, bf16, H=25, P=16 and 32; 3 / 4: end-to-end decode')
    ap.add_argument('--loop', choices=('both', 'sync', 'sync-free', 'merged'), default='both',
                    help='configs 3/4: the synchronous loop, the sync-free one (for config 4 with its graph '
                         'and merged variants), or both; config 4 merged: only the loop whose steps run '
                         'decode and replacement prefills in one layer loop')
    ap.add_argument('--prefill-each', action='store_true',
                    help='config 4: one prefill call per replaced request instead of one batched call per step')
    ap.add_argument('--replace-rate', type=float, default=0.05,
                    help='config 4: fraction of requests replaced per step (0 = decode steps only)')
    ap.add_argument('--prefill', action='store_true',
                    help='op-level causal paged prefill attention on the prompt shapes of configs 3 and 4')
    ap.add_argument('--model', choices=('gpt2-medium', 'distilgpt2'), default='gpt2-medium',
                    help='config 4: the model of the steady state (DistilGPT-2 runs in fp16, GPT-2-medium in bf16)')
    ap.add_argument('--concurrent', type=int, default=128, help='config 4: requests decoded every step')
    ap.add_argument('--projections', action='store_true',
                    help='time the decode projections (projection kernel vs hipBLASLt) at several batch sizes')
    ap.add_argument('--build-variants', action='store_true',
                    help='build the decode kernel variants (lanes per token x non-temporal loads) into '
                         'build/decode_variants/ and exit')
    ap.add_argument('--variants', action='store_true',
                    help='time the decode kernel variants x waves (4, 8) x unroll (1, 2, 4) on config 2, '
                         "config 4's layer and config 5 (P = 16)")
    ap.add_argument('--timeline', action='store_true',
                    help="per-workgroup timeline of one config-2 launch (--config 4: config 4's layer shape) "
                         'from the MT_DECODE_TIMELINE build (build it with --build-variants)')
    ap.add_argument('--entries', action='store_true',
                    help='time the decode entries (work list, batch order, mt_paged_decode_batch) on config 2 '
                         'and on one-page rows of the same shape')
    ap.add_argument('--reference-scenarios', action='store_true',
                    help="the reference's published DistilGPT-2 scenarios (serial vs continuous trace, "
                         'batch-1 paged inference at 32-512-token prompts) and its figures beside them')
    ap.add_argument('--no-config5', action='store_true',
                    help='default line: skip config 5 (ragged bf16 decode at page sizes 16 and 32)')
    ap.add_argument('--no-e2e', action='store_true',
                    help='default line: skip the end-to-end configs 3 and 4 and config 1')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: this build has no multi-GPU path '
              '(request/head sharding is a design note); run with --gpus 1.', file=sys.stderr)
        sys.exit(2)

    if args.build_variants:
        build_decode_variants()
        return
    rt = runtime()
    if args.variants:
        print(json.dumps(bench_variants(args)), flush=True)
        return
    if args.timeline:
        print(json.dumps(bench_timeline(args)), flush=True)
        return
    if args.calibrate_copy:
        from minitorch_amd.runtime import RawDeviceBuffer
        nbytes = args.calibrate_copy << 20
        src, dst = RawDeviceBuffer(nbytes), RawDeviceBuffer(nbytes)
        src.fill_words(1)
        for _ in range(args.steps):
            rt.d2d(dst.ptr, src.ptr, nbytes)
        rt.synchronize()
        print(json.dumps({'calibrate_copy_bytes': nbytes, 'copies': args.steps}), flush=True)
        return
    if args.config == 5:
        print(json.dumps(bench_config5(args)), flush=True)
        return
    if args.entries:
        print(json.dumps(bench_entries(args)), flush=True)
        return
    if args.reference_scenarios:
        print(json.dumps(reference_scenarios(args)), flush=True)
        return
    if args.prefill:
        print(json.dumps(bench_prefill(args)), flush=True)
        return
    if args.projections:
        print(json.dumps(bench_projections(args)), flush=True)
        return
    if args.config in (3, 4):
        print(json.dumps(bench_e2e(args)), flush=True)
        return
    case = config2_case(args.seed)
    devs = [DevicePagedCase(case) for _ in range(args.pools)]
    kw = devs[0].kwargs()
    split = paged_ops.split_tokens_for(page_size=case.page_size, columns=case.columns, requested=args.split)
    ws_bytes = paged_ops.decode_workspace_bytes(b=case.batch, h=case.heads, page_size=case.page_size,
                                                columns=case.columns, split_tokens=split)
    from minitorch_amd.runtime import RawDeviceBuffer
    ws = RawDeviceBuffer(max(ws_bytes, 4))
    ws.fill_words(0)
    fn = paged_ops.paged_library().mt_paged_decode_split
    fn.argtypes, fn.restype = paged_ops.SPLIT_ARGTYPES, I
    from minitorch_amd.dtypes import dtype_code
    # Work list: rows longest first, balanced over the compute units; the
    # scheduler knows the lengths on the host.
    work, items, merges = paged_ops.decode_work_list(case.lengths, case.heads, split, rt.compute_units())
    order = RawDeviceBuffer(4 * len(work))
    order.upload(work)
    work_args = (None, 0, 0) if args.natural_order else (order.ptr, items, merges)
    calls = [(d.out.ptr, d.q.ptr, d.k.ptr, d.v.ptr, d.slab_table.ptr, d.block_table.ptr, d.offsets.ptr,
              kw['b'], kw['h'], kw['d'], kw['page_size'], kw['pages_per_slab'], kw['num_slabs'],
              kw['columns'], kw['layer'], kw['layers'], dtype_code(kw['dtype']), split,
              args.unroll, args.waves, 0, *work_args, ws.ptr, ws_bytes) for d in devs]

    def step(i):
        status = fn(*calls[i % len(calls)])
        if status:
            rt.check(status)

    for i in range(args.warmup):
        step(i)
    rt.synchronize()
    start, end = CudaEvent(), CudaEvent()
    with no_gc():
        wall0 = time.perf_counter()
        start.record()
        for i in range(args.steps):
            step(i)
        end.record()
        rt.synchronize()
        wall = time.perf_counter() - wall0
    gpu_s = end.seconds_since(start)
    per_step = gpu_s / args.steps
    nbytes = algorithmic_bytes(case)
    achieved = nbytes / per_step / 1e9
    result = {
        'metric': METRIC,
        'value': case.batch / per_step,
        'unit': 'tokens/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': per_step * 1e3,
        'wall_ms_per_step': wall / args.steps * 1e3,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f16',
        'data': 'synthetic',
        'value_definition': ('op level: B requests / mean duration of ONE fused KV-append + decode-attention '
                             'launch over ONE layer (config 2); not a whole-model rate. End-to-end decode '
                             'tokens/s of full model steps: e2e.config3 / e2e.config4'),
        'config': {
            'workload': 'config 2: op-level paged decode (fused KV append + attention), B=64, '
                        'L~U[128,1024], H=12, D=64, page 16, fp16 K/V, fp32 accumulate, 8192-page '
                        'shuffled pool, cold cache via pool rotation',
            'global_batch': case.batch,
            'sum_context_tokens': int(case.lengths.sum()),
            'pools_rotated': args.pools,
            'split_tokens': split,
            'parallelism': 'single GPU',
        },
        'roofline': {
            'bound': 'hbm',
            'achieved': achieved,
            'peak': PEAK_HBM_GBS,
            'unit': 'GB/s',
            'frac': achieved / PEAK_HBM_GBS,
            'traffic': measured_traffic(),
            'traffic_source': 'profiles/decode_config2_fp16_hbm_traffic.md (rocprofv3 --pmc)',
            'algorithmic_bytes_per_launch': nbytes,
            'kernel': 'decode_kernel<kF16,64,true,U> (mt_paged_decode_split)',
        },
    }
    # the reference entry on the same pools, right after the headline timing
    # (the GPU still busy and clocked up)
    result['dropin'] = dropin_config2(case, devs, args.steps, args.warmup)
    if not args.no_ceiling:
        result['pattern_ceiling'] = pattern_ceiling(case, devs, args.steps, args.warmup)
    if not args.no_cpu_baseline:
        result['cpu_baseline'] = cpu_baseline(case, args.cpu_seconds)
    del devs, calls, ws, order
    if not args.no_config5:
        print('config 5 (page sizes 16 and 32)', file=sys.stderr, flush=True)
        c5 = bench_config5(args)
        result['config5'] = {k: c5[k] for k in ('config', 'ms_per_step', 'value', 'unit', 'roofline',
                                                'page_size_16', 'page_size_32', 'cpu_baseline')}
    if not args.no_e2e:
        print('config 1, then end-to-end configs 3 and 4', file=sys.stderr, flush=True)
        result['config1'] = config1_times(args)
        result['e2e'] = e2e_summary(e2e_config3(args), e2e_config4(args))
        print('reference scenarios', file=sys.stderr, flush=True)
        result['reference_scenarios'] = reference_scenarios(args)
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
