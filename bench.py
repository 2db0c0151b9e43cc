#!/usr/bin/env python3
"""Benchmark of the MI355X butterfly path (one GPU): every BASELINE configuration.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|c1|c2|c3a|c3b|c4|c5a|c5b|...]
                [--headline c5a] [--no-cpu] [--verify] [--eager] [--mapping LOWERING]

A step is one call of the hot path over one batch of a BASELINE configuration
(C2 and C4: forward then inverse), inputs already resident in HBM. Per
configuration: W untimed eager calls, then a HIP graph of 20 calls captured,
replayed untimed for at least 30 replays and 50 ms of GPU time (the settle
phase), and then, queued behind it with no host synchronisation in between,
replayed R = max(7, ceil(K / 20)) times, each replay bracketed by HIP events
on the plans' stream; the time per call is the MEDIAN replay / 20 (the
reference's protocol: 10 warmups, a graph of 20 calls, median of 7 replays).
The settle phase exists because on MI355X the first two dozen replays after
the GPU has idled run up to 12% slower than the rest (a clock / power
transient, e.g. C5b 46.9, 48.4, ... 52.0, then 46.2-46.9 us per call from
about the 25th replay on, whatever the eager warmup): the timed replays then
read the sustained rate at any K. The calls rotate over buffer sets whose
inputs alone exceed twice the 256 MB Infinity Cache (plus one set), so inputs
come from HBM: nontemporal output stores do not evict earlier inputs from
that cache, and a rotation sized on inputs plus outputs let C1 read part of
its input from it (20.6 against 24.0 us per call).

The default runs all seven BASELINE configurations. Rank 0 prints ONE JSON
line: the driver's fields for the headline configuration (--headline, default
C5a, one of the largest single-GPU configurations at 268 MB per call) plus
`per_config`, one entry per configuration with its roofline (algorithmic
bytes per call / median call time against 8 TB/s HBM, and the HBM traffic
counted by rocprofv3 for it) and its CPU baseline: the CPU oracle -- a C
restatement of the reference CPU path -- timed on this host at 1 thread and
at all threads, median of 7 bounded runs after one warmup.
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "transforms/s + achieved HBM GB/s (% of peak) per operator, 1x MI355X"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
CALLS_PER_GRAPH = 20
MIN_REPLAYS = 7
# Untimed graph replays queued right before the timed ones: at least this
# many, covering at least this much GPU time.
SETTLE_REPLAYS = 30
SETTLE_MS = 50.0
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
BASELINE_CONFIGS = ["c1", "c2", "c3a", "c3b", "c4", "c5a", "c5b"]
DEFAULT_HEADLINE = "c5a"

# VALU instructions per radix-2 butterfly of the NTT pass kernels, all work
# of a pass included (loads, twiddle chunks, exchanges): rocprofv3
# SQ_INSTS_VALU per dispatch divided by the dispatch's butterflies / 64,
# summed over the passes of one call. With 256 CUs x 64 lanes x 2.4 GHz this
# gives the integer-VALU roof that binds the NTT configurations before HBM.
VALU_LANE_OPS_PER_S = 256 * 64 * 2.4e9


def _device_copy(torch, a):
    view = a.view(np.int32) if a.dtype == np.uint32 else a.view(np.int64) if a.dtype == np.uint64 else a
    return torch.from_numpy(np.ascontiguousarray(view)).to("cuda")


def _rotation(input_bytes):
    """Buffer sets so that the rotated inputs alone exceed twice the Infinity
    Cache by one set: an input is read again only after that many bytes of
    other inputs."""
    return max(3, -(-2 * MALL_BYTES // max(1, input_bytes)) + 1)


class Workload:
    """One configuration: plans, rotated device buffers, a call, its bytes,
    and the CPU oracle over a slice of its rows."""

    name = ""
    dtype = ""
    description = ""
    transforms_per_call = 0
    bytes_per_call = 0  # algorithmic: compulsory input read + output write
    rows = 0            # independent transforms (rows / limbs) in one batch
    mapping = None      # --mapping: plan with this lowering (EXPLICIT)
    takes_mapping = True

    def plan_args(self):
        return {"algorithm": self.mapping} if self.mapping else {}

    def setup(self, torch, lib, stream):
        raise NotImplementedError

    def call(self, index):
        raise NotImplementedError

    def cpu_run(self, rows, threads):
        """Runs the reference CPU path over the first `rows` rows; returns
        the transforms computed."""
        raise NotImplementedError

    def kernel_name(self):
        return self.plans[0].algorithm_name()

    def _bind_workspace(self, torch, plans):
        need = max(p.workspace_size() for p in plans)
        if need:
            self.workspace = torch.empty(need, dtype=torch.uint8, device="cuda")
            for p in plans:
                if p.workspace_size():
                    p.set_workspace(self.workspace, need)

    def _rotate(self, torch, src, extra=()):
        sets = _rotation(src.numel() * src.element_size())
        self.inputs = [src.clone() for _ in range(sets)]
        self.outputs = [torch.empty_like(src) for _ in range(sets)]
        for name in extra:
            setattr(self, name, [torch.empty_like(src) for _ in range(sets)])


class OnePlan(Workload):
    """A configuration served by one plan over packed rows."""

    def descriptor(self, cb):
        raise NotImplementedError

    def make_host(self):
        raise NotImplementedError

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        self.plans = [cb.Plan(lib, self.descriptor(cb), stream=stream, **self.plan_args())]
        self._bind_workspace(torch, self.plans)
        self.host = self.make_host()
        self._rotate(torch, _device_copy(torch, self.host))

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.outputs[k])


class FwhtFp32(OnePlan):
    name, dtype = "c1", "f32"

    def __init__(self, log_n=12, batch=4096):
        self.log_n, self.rows = log_n, batch
        self.description = f"C1: FWHT fp32 unnormalized forward, batch {batch} x n={1 << log_n}, integer inputs in [-8,8]"
        self.transforms_per_call = batch
        self.bytes_per_call = 2 * batch * (4 << log_n)

    def descriptor(self, cb):
        return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1 << self.log_n], self.rows,
                           compute=cb.ComputeType.FP32)

    def make_host(self):
        from cubutterfly_amd import workloads
        return workloads.fwht_integer_input(self.log_n, self.rows, seed=1)

    def verify(self):
        import oracle
        got = self.outputs[0].cpu().numpy()
        return bool(np.array_equal(got, oracle.fwht_f32(self.host, threads=oracle.default_threads())))

    def cpu_run(self, rows, threads):
        import oracle
        oracle.fwht_f32(self.host[:rows], threads=threads)
        return rows


class FwhtFp32Pitched(FwhtFp32):
    """C1's transform on rows pitched by n + 64 on both sides (not a BASELINE
    line): the FWHT kernel reads and writes the pitched rows directly."""
    name = "c1p"
    PAD = 64

    def __init__(self, log_n=12, batch=4096):
        super().__init__(log_n, batch)
        self.description = "C1 on rows pitched at n + 64 elements on both sides (pitched-row FWHT kernel)"

    def descriptor(self, cb):
        n = 1 << self.log_n
        pitch = n + self.PAD
        return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], self.rows, compute=cb.ComputeType.FP32,
                           input_strides=[1], input_batch_stride=pitch, output_strides=[1],
                           output_batch_stride=pitch)

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        from cubutterfly_amd import workloads
        n = 1 << self.log_n
        pitch = n + self.PAD
        self.plans = [cb.Plan(lib, self.descriptor(cb), stream=stream, **self.plan_args())]
        self._bind_workspace(torch, self.plans)
        self.host = workloads.fwht_integer_input(self.log_n, self.rows, seed=1)
        padded = np.zeros((self.rows, pitch), dtype=np.float32)
        padded[:, :n] = self.host
        flat = padded.reshape(-1)[: (self.rows - 1) * pitch + n]
        self._rotate(torch, _device_copy(torch, flat))

    def verify(self):
        import oracle
        n, pitch = 1 << self.log_n, (1 << self.log_n) + self.PAD
        flat = self.outputs[0].cpu().numpy()
        got = np.zeros(self.rows * pitch, dtype=np.float32)
        got[: flat.size] = flat
        got = got.reshape(self.rows, pitch)[:, :n]
        return bool(np.array_equal(got, oracle.fwht_f32(self.host, threads=oracle.default_threads())))


class NttNegacyclic(Workload):
    """C2: forward then inverse negacyclic NTT, u32, q = 1073479681, n = 2^16, batch 64."""
    name, dtype = "c2", "u32"
    valu_per_butterfly = 8.6

    def __init__(self, log_n=16, batch=64):
        from cubutterfly_amd import workloads
        self.log_n, self.rows, self.q = log_n, batch, workloads.C2_MODULUS
        self.description = (f"C2: single-prime negacyclic NTT u32, n=2^{log_n}, batch {batch}, q=1073479681 (30-bit, "
                            "q = 1 mod 2n); one step = forward then inverse of the batch")
        self.transforms_per_call = 2 * batch  # forward + inverse transforms
        self.bytes_per_call = 2 * 2 * batch * (4 << log_n)
        self.butterflies_per_call = self.transforms_per_call * (1 << (log_n - 1)) * log_n

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        from cubutterfly_amd import workloads

        def plan(inverse):
            d = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [1 << self.log_n], self.rows,
                            compute=cb.ComputeType.UINT32, modulus=self.q, word_bits=32, inverse=inverse,
                            ntt_ring=cb.NttRing.NEGACYCLIC)
            return cb.Plan(lib, d, stream=stream, **self.plan_args())

        self.plans = [plan(False), plan(True)]
        self._bind_workspace(torch, self.plans)
        self.host = workloads.ntt_input(self.log_n, self.rows, self.q, seed=1).astype(np.uint32)
        src = _device_copy(torch, self.host)
        self._rotate(torch, src, extra=("spectra",))

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.spectra[k])
        self.plans[1].execute(self.spectra[k], self.outputs[k])

    def verify(self):
        import oracle
        spectrum = self.spectra[0].cpu().numpy().view(np.uint32).astype(np.uint64)
        back = self.outputs[0].cpu().numpy().view(np.uint32)
        expected = oracle.ntt_negacyclic(self.host.astype(np.uint64), self.q, threads=oracle.default_threads())
        return bool(np.array_equal(spectrum, expected) and np.array_equal(back, self.host))

    def kernel_name(self):
        return self.plans[0].algorithm_name() + " (forward) + inverse"

    def cpu_run(self, rows, threads):
        import oracle
        y = oracle.ntt_negacyclic(self.host[:rows].astype(np.uint64), self.q, threads=threads)
        oracle.ntt_negacyclic(y, self.q, inverse=True, threads=threads)
        return 2 * rows


class RnsNegacyclic(Workload):
    """C4: RNS negacyclic NTT, 32 limbs x n = 2^16 of 60-bit primes, forward
    (natural -> bit-reversed) then inverse (bit-reversed -> natural)."""
    name, dtype = "c4", "u64"
    description = ("C4: RNS negacyclic NTT u64, n=2^16, 32 limbs of distinct 60-bit primes (q = 1 mod 2^17), "
                   "one step = forward (natural->bit_reversed) then inverse (bit_reversed->natural)")
    valu_per_butterfly = 26.1
    takes_mapping = False

    def __init__(self, log_n=16, limbs=32):
        from cubutterfly_amd import workloads
        self.log_n, self.rows = log_n, limbs
        self.moduli = workloads.c4_moduli()[:limbs]
        self.transforms_per_call = 2 * limbs
        self.bytes_per_call = 2 * 2 * limbs * (8 << log_n)
        self.butterflies_per_call = self.transforms_per_call * (1 << (log_n - 1)) * log_n

    def setup(self, torch, lib, stream):
        from cubutterfly_amd import ntt_roots, rns, workloads
        # psi_i: the reference's rule, smallest-candidate primitive 2n-th root.
        self.roots = [ntt_roots.primitive_root(self.log_n + 1, q) for q in self.moduli]
        domains = list(zip(self.moduli, self.roots))
        self.plans = []
        for inverse in (False, True):
            plan = rns.RnsPlan(lib, rns.request(self.log_n, domains, inverse=inverse))
            plan.prepare(stream, repetitions=3)
            self.plans.append(plan)
        self.stream = stream
        self.host = np.stack([workloads.ntt_input(self.log_n, 1, q, seed=1, channel=i)[0]
                              for i, q in enumerate(self.moduli)])
        src = _device_copy(torch, self.host)
        self._rotate(torch, src, extra=("spectra",))

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.spectra[k], self.stream)
        self.plans[1].execute(self.spectra[k], self.outputs[k], self.stream)

    def verify(self):
        import oracle
        spectrum = self.spectra[0].cpu().numpy().view(np.uint64)
        back = self.outputs[0].cpu().numpy().view(np.uint64)
        expected = oracle.rns(self.host, self.moduli, self.roots, output_bit_reversed=True,
                              threads=oracle.default_threads())
        return bool(np.array_equal(spectrum, expected) and np.array_equal(back, self.host))

    def kernel_name(self):
        return self.plans[0].info()["mapping"]["algorithm"] + " (forward) + inverse"

    def cpu_run(self, rows, threads):
        import oracle
        y = oracle.rns(self.host[:rows], self.moduli[:rows], self.roots[:rows], output_bit_reversed=True,
                       threads=threads)
        oracle.rns(y, self.moduli[:rows], self.roots[:rows], inverse=True, input_bit_reversed=True,
                   threads=threads)
        return 2 * rows


class FftC64(OnePlan):
    """C3: complex64 FFT forward, 1 x 2^24 (c3a) or 1024 x 2^14 (c3b)."""
    dtype = "c64"

    def __init__(self, log_n, batch):
        self.log_n, self.rows = log_n, batch
        self.name = "c3a" if batch == 1 else "c3b"
        self.description = (f"{self.name.upper()}: complex FFT c64 forward, batch {batch} x n=2^{log_n}, "
                            "N(0,1) real and imaginary parts")
        self.transforms_per_call = batch
        self.bytes_per_call = 2 * batch * (8 << log_n)

    def descriptor(self, cb):
        return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << self.log_n], self.rows,
                           compute=cb.ComputeType.FP32)

    def make_host(self):
        from cubutterfly_amd import workloads
        return workloads.complex_input(self.log_n, self.rows, seed=3).reshape(self.rows, 1 << self.log_n)

    def verify(self):
        import oracle
        got = self.outputs[0].cpu().numpy().astype(np.complex128)
        ref = oracle.fft_c64(self.host, threads=oracle.default_threads()).astype(np.complex128)
        err = np.linalg.norm(got - ref, axis=-1) / np.linalg.norm(ref, axis=-1)
        return bool(np.max(err) <= 1e-5)

    def cpu_run(self, rows, threads):
        import oracle
        oracle.fft_c64(self.host[:rows], threads=threads)
        return rows


class FftC64Rank2(FftC64):
    """Rank-2 complex64 FFT, 4096 x 4096 (not a BASELINE line)."""

    def __init__(self):
        super().__init__(24, 1)
        self.name = "r2"
        self.description = "rank-2 complex FFT c64 forward, 4096 x 4096, batch 1, N(0,1) parts"

    def descriptor(self, cb):
        return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [4096, 4096], 1, compute=cb.ComputeType.FP32)

    def verify(self):
        got = self.outputs[0].cpu().numpy().reshape(4096, 4096).astype(np.complex128)
        ref = np.fft.fft2(self.host.reshape(4096, 4096).astype(np.complex128))
        return bool(np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5)

    def cpu_run(self, rows, threads):
        import oracle
        first = oracle.fft_c64(self.host.reshape(4096, 4096), threads=threads)
        oracle.fft_c64(np.ascontiguousarray(first.T), threads=threads)
        return 1


class FwhtFp16(OnePlan):
    """C5: QuaRot-style FP16 FWHT, scale 1/sqrt(n), FP32 compute, one final
    FP16 rounding: 16384 x 4096 (c5a) or 524288 x 128 (c5b)."""
    dtype = "f16"

    def __init__(self, rows, n, mma=False):
        self.rows, self.n, self.mma = rows, n, mma
        self.name = ("c5a" if n == 4096 else "c5b") + ("_mma" if mma else "")
        self.description = (f"{self.name.upper()}: FWHT fp16 storage / fp32 compute, {rows} x n={n}, output scale "
                            "1/sqrt(n), final-storage rounding, N(0,1) activations with x50 outlier channels"
                            + (", ALLOW_FP16_MMA (MFMA 16x16 Hadamard blocks; not the bit-exact default)"
                               if mma else ""))
        self.transforms_per_call = rows
        self.bytes_per_call = 2 * rows * n * 2
        self.scale = float(np.float32(1.0 / np.sqrt(n)))

    def plan_args(self):
        # The MFMA lowering is taken by name (ALLOW_FP16_MMA keeps the
        # stage-ordered kernel as its default).
        if self.mma and not self.mapping:
            return {"algorithm": "fwht-fp16-mfma16"}
        return super().plan_args()

    def descriptor(self, cb):
        policy = cb.ArithmeticPolicy.ALLOW_FP16_MMA if self.mma else cb.ArithmeticPolicy.STRICT
        return cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [self.n], self.rows, compute=cb.ComputeType.FP32,
                           output_scale=self.scale, output_rounding=cb.OutputRounding.FINAL_STORAGE,
                           arithmetic_policy=policy)

    def make_host(self):
        from cubutterfly_amd import workloads
        return workloads.quarot_input(self.rows, self.n, seed=5)

    def verify(self):
        import oracle
        got = self.outputs[0].cpu().numpy().view(np.float16).astype(np.float32)
        ref16 = oracle.fwht_f16_final(self.host, self.scale, threads=oracle.default_threads())
        ref = ref16.astype(np.float32)
        if self.mma:  # within 2e-3 or one fp16 ulp of the oracle (different accumulation order)
            return bool(np.all(np.abs(got - ref) <= np.maximum(2e-3, np.spacing(np.abs(ref16)).astype(np.float32))))
        return bool(np.max(np.abs(got - ref)) <= 2e-3)

    def cpu_run(self, rows, threads):
        import oracle
        oracle.fwht_f16_final(self.host[:rows], self.scale, threads=threads)
        return rows


class DeviceCopy(Workload):
    """Calibration probe, not a BASELINE config: a plain device-to-device copy
    of 128 MiB, the known-size reference for rocprofv3 FETCH_SIZE/WRITE_SIZE."""
    name, dtype = "copy", "u8"
    description = "plain device copy of 134217728 bytes (HBM traffic counter calibration)"
    transforms_per_call = 1
    bytes_per_call = 2 * 134217728
    takes_mapping = False

    def setup(self, torch, lib, stream):
        self._rotate(torch, torch.ones(134217728 // 4, dtype=torch.float32, device="cuda"))

    def call(self, index):
        k = index % len(self.inputs)
        self.outputs[k].copy_(self.inputs[k])

    def kernel_name(self):
        return "torch copy_"


class FwhtFp32Long(FwhtFp32):
    """C1's 64 MiB as rows of 2^16 points (not a BASELINE line): the factored
    plan, a resident row pass and one in-place column pass."""
    name = "c1l"

    def __init__(self, log_n=16, batch=256):
        super().__init__(log_n, batch)
        self.description = (f"FWHT fp32 unnormalized forward, batch {batch} x n={1 << log_n} (factored: a resident "
                            "row pass and an in-place column pass), integer inputs in [-8,8]")


WORKLOADS = {"c1": FwhtFp32, "c1p": FwhtFp32Pitched, "c1l": FwhtFp32Long, "c2": NttNegacyclic, "c3a": lambda: FftC64(24, 1),
             "c3b": lambda: FftC64(14, 1024), "c4": RnsNegacyclic, "c5a": lambda: FwhtFp16(16384, 4096),
             "c5b": lambda: FwhtFp16(524288, 128), "c5a_mma": lambda: FwhtFp16(16384, 4096, mma=True),
             "c5b_mma": lambda: FwhtFp16(524288, 128, mma=True), "r2": FftC64Rank2, "copy": DeviceCopy}


# Configurations whose batch (rows, polynomials) `--batch` can change, for
# sweeps that separate a kernel's fixed cost from its per-row rate.
BATCHED = {"c1": lambda b: FwhtFp32(12, b), "c2": lambda b: NttNegacyclic(16, b), "c3b": lambda b: FftC64(14, b),
           "c5a": lambda b: FwhtFp16(b, 4096), "c5b": lambda b: FwhtFp16(b, 128)}


def measured_traffic(name):
    """HBM bytes per call (read, write) for a configuration, from the
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary in profiles/ (scaled by the copy
    calibration recorded there), or None when no measurement exists."""
    try:
        with open(TRAFFIC_TABLE) as f:
            for line in f:
                fields = line.split()
                if len(fields) == 3 and fields[0] == name:
                    return int(fields[1]), int(fields[2])
    except OSError:
        pass
    return None


def time_graph_replays(torch, workload, stream, steps, warmup):
    """Per-call milliseconds of each replay of a 20-call graph (the median is
    the reported figure) and the number of timed calls."""
    with torch.cuda.stream(stream):
        for i in range(warmup):
            workload.call(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(CALLS_PER_GRAPH):
            workload.call(i)
    torch.cuda.synchronize()
    replays = max(MIN_REPLAYS, -(-steps // CALLS_PER_GRAPH))
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        graph.replay()  # the first replay uploads the graph
        torch.cuda.synchronize()
        # One replay timed alone sizes the settle phase.
        probe = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        probe[0].record(stream)
        graph.replay()
        probe[1].record(stream)
        torch.cuda.synchronize()
        replay_ms = max(probe[0].elapsed_time(probe[1]), 1e-3)
        settle = max(SETTLE_REPLAYS, int(SETTLE_MS / replay_ms) + 1)
        # Untimed replays, then the timed ones, queued back to back with no
        # host synchronisation in between: the GPU never idles before the
        # timed region, so it is measured past the post-idle clock transient.
        for _ in range(settle):
            graph.replay()
        for start, stop in marks:
            start.record(stream)
            graph.replay()
            stop.record(stream)
    torch.cuda.synchronize()
    per_call = [start.elapsed_time(stop) / CALLS_PER_GRAPH for start, stop in marks]
    del graph
    return per_call, replays * CALLS_PER_GRAPH


def time_eager(torch, workload, stream, steps, warmup):
    with torch.cuda.stream(stream):
        for i in range(warmup):
            workload.call(i)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    with torch.cuda.stream(stream):
        for i in range(steps):
            workload.call(warmup + i)
    stop.record(stream)
    torch.cuda.synchronize()
    return [start.elapsed_time(stop) / steps], steps


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_rate(workload, threads, target_s=0.25, reps=7):
    """Transforms/s of the CPU oracle over a bounded slice of the workload's
    rows: the slice is sized to about `target_s` per run; one warmup, then the
    median of `reps` runs (3 runs and no warmup when one row alone takes more
    than a second). Returns (rate, sample description)."""
    total = workload.rows
    rows = max(1, min(total, threads))
    t0 = time.perf_counter()
    workload.cpu_run(rows, threads)
    elapsed = time.perf_counter() - t0
    while elapsed < 0.02 and rows < total:
        rows = min(total, rows * 4)
        t0 = time.perf_counter()
        workload.cpu_run(rows, threads)
        elapsed = time.perf_counter() - t0
    slow = elapsed > 1.0
    if not slow:
        rows = max(1, min(total, int(rows * target_s / elapsed)))
        if rows >= threads:
            rows -= rows % threads
        workload.cpu_run(rows, threads)  # warmup at the sampled size
    runs = 3 if slow else reps
    times, transforms = [], 0
    for _ in range(runs):
        t0 = time.perf_counter()
        transforms = workload.cpu_run(rows, threads)
        times.append(time.perf_counter() - t0)
    median = statistics.median(times)
    sample = (f"{rows} of {total} rows per run, median of {runs} runs" + ("" if slow else " after 1 warmup")
              + f", {threads} thread{'s' if threads > 1 else ''}, {median * 1e3:.1f} ms per run")
    return transforms / median, sample


def measure(torch, lib, name, args, mapping=None):
    """Times one configuration on the GPU; returns its per_config entry."""
    batch = getattr(args, "batch", None)
    workload = BATCHED[name](batch) if batch else WORKLOADS[name]()
    if mapping:
        if not workload.takes_mapping:
            raise SystemExit(f"--mapping does not apply to {name}")
        workload.mapping = mapping
    stream = torch.cuda.Stream()  # default priority; plans launch on it
    workload.setup(torch, lib, stream.cuda_stream)
    torch.cuda.synchronize()
    timer = time_eager if args.eager else time_graph_replays
    per_call, timed = timer(torch, workload, stream, args.steps, args.warmup)
    ms = statistics.median(per_call)
    achieved = workload.bytes_per_call / (ms * 1e-3) / 1e9
    traffic = None if batch else measured_traffic(name)  # the summaries are per BASELINE shape
    entry = {
        "config": name if not batch else f"{name}@batch={batch}",
        "workload": workload.description,
        "dtype": workload.dtype,
        "kernel": workload.kernel_name(),
        "ms_per_call": ms,
        # The reference's protocol reading: the median of the first 7 replays.
        "ms_per_call_first7": statistics.median(per_call[:MIN_REPLAYS]),
        "ms_per_call_replays": per_call,
        "timed_calls": timed,
        "transforms_per_call": workload.transforms_per_call,
        "transforms_per_s": workload.transforms_per_call / (ms * 1e-3),
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None if traffic is None else sum(traffic),
            "traffic_read_write": traffic,
            "algorithmic_bytes_per_call": workload.bytes_per_call,
        },
    }
    if traffic is not None:
        entry["roofline"]["traffic_over_algorithmic"] = sum(traffic) / workload.bytes_per_call
    if hasattr(workload, "valu_per_butterfly"):
        rate = workload.butterflies_per_call / (ms * 1e-3)
        peak = VALU_LANE_OPS_PER_S / workload.valu_per_butterfly
        entry["valu_roofline"] = {"bound": "valu", "achieved": rate, "peak": peak, "unit": "butterflies/s",
                                  "frac": rate / peak, "valu_per_butterfly": workload.valu_per_butterfly,
                                  "floor_ms_per_call": workload.butterflies_per_call / peak * 1e3}
    if args.verify and hasattr(workload, "verify"):
        entry["verified"] = workload.verify()
    # Device buffers go before the CPU leg and the next configuration.
    for attr in ("inputs", "outputs", "spectra", "workspace"):
        if hasattr(workload, attr):
            delattr(workload, attr)
    for plan in getattr(workload, "plans", []):
        plan.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not args.no_cpu and hasattr(workload, "host"):
        import oracle
        threads = oracle.default_threads()
        one, one_sample = cpu_rate(workload, 1)
        entry["cpu_baseline"] = {"value_1core": one, "sample_1core": one_sample, "unit": "transforms/s",
                                 "kind": "port", "cpu_model": cpu_model()}
        if workload.rows > 1 and threads > 1:
            many, many_sample = cpu_rate(workload, threads)
            entry["cpu_baseline"].update(value=many, cores=threads, sample=many_sample)
        else:
            entry["cpu_baseline"].update(value=one, cores=1, sample=one_sample + " (one transform: 1 core only)")
    print(f"# {entry['config']}: {ms * 1e3:.2f} us per call, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%}); "
          f"median of the first {MIN_REPLAYS} replays {entry['ms_per_call_first7'] * 1e3:.2f} us",
          file=sys.stderr, flush=True)
    return entry


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=1200)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default="all", choices=["all"] + sorted(WORKLOADS))
    parser.add_argument("--headline", default=DEFAULT_HEADLINE, choices=BASELINE_CONFIGS)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    parser.add_argument("--verify", action="store_true", help="check each output against the oracle")
    parser.add_argument("--eager", action="store_true", help="time eager submissions instead of graph replays")
    parser.add_argument("--mapping", default=None, help="plan a single --workload with this lowering (EXPLICIT)")
    parser.add_argument("--batch", type=int, default=None,
                        help="rows / polynomials of a single --workload (" + " ".join(sorted(BATCHED)) + ")")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every configuration of the butterfly path runs on one GPU and "
              "shards by rows or limbs without communication; multi-GPU runs are not part of this build",
              file=sys.stderr)
        sys.exit(2)
    if args.mapping and args.workload == "all":
        print("--mapping needs a single --workload", file=sys.stderr)
        sys.exit(2)
    if args.batch is not None and (args.workload not in BATCHED or args.batch < 1):
        print("--batch needs a single --workload among " + ", ".join(sorted(BATCHED)) + " and a positive count",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import cubutterfly_amd as cb
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    lib = cb.Native()
    names = BASELINE_CONFIGS if args.workload == "all" else [args.workload]
    entries = [measure(torch, lib, name, args, args.mapping) for name in names]
    head = next((e for e in entries if e["config"] == args.headline), entries[0])
    result = {
        "metric": METRIC,
        "value": head["transforms_per_s"],
        "unit": "transforms/s",
        "n_gpus": 1,
        "steps": head["timed_calls"],
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded splitmix64 / mt19937_64 generators)",
        "config": {"workload": head["workload"], "headline": head["config"],
                   "configs_measured": [e["config"] for e in entries]},
        "roofline": dict(head["roofline"], kernel=head["kernel"]),
        "timing": ("eager calls" if args.eager else
                   f"median of {len(head['ms_per_call_replays'])} replays of a HIP graph of {CALLS_PER_GRAPH} "
                   f"calls, HIP events on the plans' stream, after an untimed settle phase of at least "
                   f"{SETTLE_REPLAYS} replays and {SETTLE_MS:.0f} ms queued back to back with the timed replays "
                   f"(ms_per_call_first7: the median of the first {MIN_REPLAYS} timed replays, the reference's "
                   "protocol)"),
        "per_config": entries,
    }
    if "cpu_baseline" in head:
        result["cpu_baseline"] = head["cpu_baseline"]
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
