#!/usr/bin/env python3
"""Headline benchmark of the MI355X butterfly path (one GPU).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c1|c1p|c2|c3a|c3b|c4|c5a|c5b|r2|copy]
                [--no-cpu] [--verify] [--eager] [--mapping LOWERING]

A step is one call of the hot path over one batch of the named BASELINE
configuration, with inputs already resident in HBM. W untimed steps, then K
timed steps bracketed by torch.cuda.synchronize(); the timed calls rotate over
enough input/output buffer sets (> 256 MiB in total) that the 256 MB Infinity
Cache cannot serve them. Rank 0 prints ONE JSON line with the driver's fields
plus `roofline` (algorithmic bytes per call / measured call time vs 8 TB/s HBM)
and `cpu_baseline` (the CPU oracle -- a restatement of the reference CPU path --
timed on this host over a bounded sample of the same workload).
--mapping plans the workload with the EXPLICIT policy and the named lowering
(c1, c1p, c2 and the one-plan workloads), for comparing lowerings.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "transforms/s + achieved HBM GB/s (% of peak) per operator, 1x MI355X"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def _np_to_torch(torch, a):
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(np.ascontiguousarray(a))


class Workload:
    """One BASELINE configuration: plans, resident buffers, a call, its bytes."""

    name = ""
    dtype = ""
    description = ""
    transforms_per_call = 0
    bytes_per_call = 0  # algorithmic: compulsory input read + output write

    def setup(self, torch, lib, stream):
        raise NotImplementedError

    def call(self, index):
        raise NotImplementedError

    def cpu_sample(self, threads):
        """Returns (seconds, transforms, description) for a bounded CPU run."""
        raise NotImplementedError

    def config(self):
        return {"workload": self.description}

    def kernel_name(self):
        return self.plans[0].algorithm_name()

    # --mapping: a lowering name to plan with the EXPLICIT policy, for the
    # workloads whose setup honours it (one plan per call).
    mapping = None
    takes_mapping = False

    def plan_options(self, cb):
        return cb.PlanOptions(policy=cb.AlgorithmPolicy.EXPLICIT, mapping=self.mapping) if self.mapping else None

    def _rotation(self, torch, bytes_per_set):
        return max(3, -(-2 * MALL_BYTES // max(1, bytes_per_set)))


class FwhtFp32(Workload):
    name = "c1"
    dtype = "f32"
    takes_mapping = True
    description = "FWHT fp32 unnormalized forward, batch 4096 x n=4096, integer inputs in [-8,8]"

    def __init__(self, log_n=12, batch=4096):
        self.log_n, self.batch = log_n, batch
        self.transforms_per_call = batch
        self.bytes_per_call = 2 * batch * (4 << log_n)

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        from cubutterfly_amd import workloads
        t = cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP32, compute=cb.ComputeType.FP32,
                         extents=[1 << self.log_n], batch=self.batch)
        self.plans = [cb.Plan(lib, t, options=self.plan_options(cb), stream=stream)]
        host = workloads.fwht_integer_input(self.log_n, self.batch, seed=1)
        self.host = host
        sets = self._rotation(torch, self.bytes_per_call)
        src = _np_to_torch(torch, host).to("cuda")
        self.inputs = [src.clone() for _ in range(sets)]
        self.outputs = [torch.empty_like(src) for _ in range(sets)]

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.outputs[k])

    def verify(self, torch):
        import oracle
        got = self.outputs[0].cpu().numpy()
        return bool(np.array_equal(got, oracle.fwht_f32(self.host, threads=oracle.default_threads())))

    def cpu_sample(self, threads):
        import oracle
        reps, elapsed = 0, 0.0
        while elapsed < 10.0:
            t0 = time.perf_counter()
            oracle.fwht_f32(self.host, threads=threads)
            elapsed += time.perf_counter() - t0
            reps += 1
        return elapsed, reps * self.batch, f"{reps} full C1 batches (4096 x 4096) through reference_fwht"


class FwhtFp32Pitched(FwhtFp32):
    """C1's transform on pitched rows (row stride n + 64 on both sides): the
    FWHT kernel reads and writes the pitched rows directly."""
    name = "c1p"
    description = ("FWHT fp32 unnormalized forward, batch 4096 x n=4096, rows pitched at n + 64 on both sides "
                   "(pitched-row FWHT kernel), integer inputs in [-8,8]")
    PAD = 64

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        from cubutterfly_amd import workloads
        n = 1 << self.log_n
        pitch = n + self.PAD
        t = cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP32, compute=cb.ComputeType.FP32,
                         extents=[n], batch=self.batch, input_strides=[1], input_batch_stride=pitch,
                         output_strides=[1], output_batch_stride=pitch)
        plan = cb.Plan(lib, t, options=self.plan_options(cb), stream=stream)
        ws = plan.workspace_size()
        if ws:
            self.workspace = torch.empty(ws, dtype=torch.uint8, device="cuda")
            plan.set_workspace(self.workspace, ws)
        self.plans = [plan]
        self.host = workloads.fwht_integer_input(self.log_n, self.batch, seed=1)
        padded = np.zeros((self.batch, pitch), dtype=np.float32)
        padded[:, :n] = self.host
        flat = padded.reshape(-1)[: (self.batch - 1) * pitch + n]
        sets = self._rotation(torch, self.bytes_per_call)
        src = _np_to_torch(torch, np.ascontiguousarray(flat)).to("cuda")
        self.inputs = [src.clone() for _ in range(sets)]
        self.outputs = [torch.zeros_like(src) for _ in range(sets)]

    def verify(self, torch):
        import oracle
        n, pitch = 1 << self.log_n, (1 << self.log_n) + self.PAD
        flat = self.outputs[0].cpu().numpy()
        got = np.zeros((self.batch, pitch), dtype=np.float32).reshape(-1)
        got[: flat.size] = flat
        got = got.reshape(self.batch, pitch)[:, :n]
        return bool(np.array_equal(got, oracle.fwht_f32(self.host, threads=oracle.default_threads())))

    def kernel_name(self):
        name = self.plans[0].algorithm_name()
        kernel = ("fwht_wide_kernel" if "-r32" in name else
                  "fwht_pitched_kernel" if name.endswith("-pitched") else "fwht_resident_kernel")
        return kernel + " (inside " + name + ")"


# VALU instructions per radix-2 butterfly of the NTT pass kernels, all work
# of a pass included (loads, twiddle chunks, exchanges): rocprofv3
# SQ_INSTS_VALU per dispatch divided by the dispatch's butterflies / 64,
# summed over the four passes of one call (u32 lazy: 8.6; u64 lazy: 26.1).
# With 256 CUs x 64 lanes x 2.4 GHz this gives the integer-VALU roof that
# binds the NTT configs before HBM does.
VALU_LANE_OPS_PER_S = 256 * 64 * 2.4e9


class NttNegacyclic(Workload):
    """C2: forward then inverse negacyclic NTT, u32, q = 1073479681, n = 2^16, batch 64."""
    name = "c2"
    dtype = "u32"
    description = ("single-prime negacyclic NTT u32, n=2^16, batch 64, q=1073479681 (30-bit, q = 1 mod 2n); "
                   "one step = forward then inverse of the batch")

    valu_per_butterfly = 8.6
    takes_mapping = True  # both plans (the lowering names do not depend on the direction)

    def __init__(self, log_n=16, batch=64):
        from cubutterfly_amd import workloads
        self.log_n, self.batch, self.q = log_n, batch, workloads.C2_MODULUS
        self.transforms_per_call = 2 * batch  # forward + inverse transforms
        self.bytes_per_call = 2 * 2 * batch * (4 << log_n)
        self.butterflies_per_call = self.transforms_per_call * (1 << (log_n - 1)) * log_n

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        from cubutterfly_amd import workloads

        def plan(inverse):
            t = cb.Transform(op=cb.Operator.NTT, storage=cb.DataType.UINT32, compute=cb.ComputeType.UINT32,
                             extents=[1 << self.log_n], batch=self.batch, modulus=self.q, word_bits=32,
                             inverse=inverse, ring=cb.NttRing.NEGACYCLIC)
            return cb.Plan(lib, t, options=self.plan_options(cb), stream=stream)

        self.plans = [plan(False), plan(True)]
        ws_bytes = max(p.workspace_size() for p in self.plans)
        self.workspace = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
        for p in self.plans:
            if p.workspace_size():
                p.set_workspace(self.workspace, ws_bytes)
        self.host = workloads.ntt_input(self.log_n, self.batch, self.q, seed=1).astype(np.uint32)
        src = _np_to_torch(torch, self.host).to("cuda")
        sets = self._rotation(torch, 3 * src.numel() * 4)
        self.inputs = [src.clone() for _ in range(sets)]
        self.spectra = [torch.empty_like(src) for _ in range(sets)]
        self.outputs = [torch.empty_like(src) for _ in range(sets)]

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.spectra[k])
        self.plans[1].execute(self.spectra[k], self.outputs[k])

    def verify(self, torch):
        import oracle
        spectrum = self.spectra[0].cpu().numpy().view(np.uint32).astype(np.uint64)
        back = self.outputs[0].cpu().numpy().view(np.uint32)
        expected = oracle.ntt_negacyclic(self.host.astype(np.uint64), self.q, threads=oracle.default_threads())
        return bool(np.array_equal(spectrum, expected) and np.array_equal(back, self.host))

    def kernel_name(self):
        return self.plans[0].algorithm_name() + " (forward) + inverse"

    def cpu_sample(self, threads):
        import oracle
        x = self.host.astype(np.uint64)
        reps, elapsed = 0, 0.0
        while elapsed < 10.0:
            t0 = time.perf_counter()
            y = oracle.ntt_negacyclic(x, self.q, threads=threads)
            oracle.ntt_negacyclic(y, self.q, inverse=True, threads=threads)
            elapsed += time.perf_counter() - t0
            reps += 1
        return elapsed, reps * 2 * self.batch, (f"{reps} full C2 steps (64 x 2^16 forward + inverse) through the "
                                                "crypto-benchmark composition: psi twist + reference_ntt DIT")


class RnsNegacyclic(Workload):
    """C4: RNS negacyclic NTT, 32 limbs x n = 2^16 of 60-bit primes, forward
    (natural -> bit-reversed) then inverse (bit-reversed -> natural)."""
    name = "c4"
    dtype = "u64"
    description = ("RNS negacyclic NTT u64, n=2^16, 32 limbs of distinct 60-bit primes (q = 1 mod 2^17), "
                   "one step = forward (natural->bit_reversed) then inverse (bit_reversed->natural)")

    valu_per_butterfly = 26.1
    def __init__(self, log_n=16, limbs=32):
        from cubutterfly_amd import workloads
        self.log_n, self.limbs = log_n, limbs
        self.moduli = workloads.c4_moduli()[:limbs]
        self.transforms_per_call = 2 * limbs
        self.bytes_per_call = 2 * 2 * limbs * (8 << log_n)
        self.butterflies_per_call = self.transforms_per_call * (1 << (log_n - 1)) * log_n

    def setup(self, torch, lib, stream):
        from cubutterfly_amd import ntt_roots, rns, workloads
        rlib = rns.Library()
        # psi_i: the reference's rule, smallest-candidate primitive 2n-th root.
        self.roots = [ntt_roots.primitive_root(self.log_n + 1, q) for q in self.moduli]
        domains = list(zip(self.moduli, self.roots))
        self.plans = []
        for inverse in (False, True):
            plan = rns.Plan(rlib, rns.config(self.log_n, domains, inverse=inverse))
            plan.prepare(placement=rns.Placement.SEPARATE, stream=stream, repetitions=3)
            self.plans.append(plan)
        self.stream = stream
        self.host = np.stack([workloads.ntt_input(self.log_n, 1, q, seed=1, channel=i)[0]
                              for i, q in enumerate(self.moduli)])
        src = _np_to_torch(torch, self.host).to("cuda")
        sets = self._rotation(torch, 3 * src.numel() * 8)
        self.inputs = [src.clone() for _ in range(sets)]
        self.spectra = [torch.empty_like(src) for _ in range(sets)]
        self.outputs = [torch.empty_like(src) for _ in range(sets)]

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.spectra[k], stream=self.stream)
        self.plans[1].execute(self.spectra[k], self.outputs[k], stream=self.stream)

    def verify(self, torch):
        import oracle
        spectrum = self.spectra[0].cpu().numpy().view(np.uint64)
        back = self.outputs[0].cpu().numpy().view(np.uint64)
        expected = oracle.rns(self.host, self.moduli, self.roots, output_bit_reversed=True,
                              threads=oracle.default_threads())
        return bool(np.array_equal(spectrum, expected) and np.array_equal(back, self.host))

    def kernel_name(self):
        return self.plans[0].info()["mapping"]["algorithm"] + " (forward) + inverse"

    def cpu_sample(self, threads):
        import oracle
        reps, elapsed = 0, 0.0
        while elapsed < 10.0:
            t0 = time.perf_counter()
            y = oracle.rns(self.host, self.moduli, self.roots, output_bit_reversed=True, threads=threads)
            oracle.rns(y, self.moduli, self.roots, inverse=True, input_bit_reversed=True, threads=threads)
            elapsed += time.perf_counter() - t0
            reps += 1
        return elapsed, reps * 2 * self.limbs, (f"{reps} full C4 steps (32 limbs x 2^16 forward + inverse) through "
                                                "the reference RNS oracle (tests/test_rns_ntt.cu:62-111)")


class OnePlan(Workload):
    """A configuration served by one plan: host input -> rotated device sets."""

    elem_bytes = 0

    def transform(self, cb):
        raise NotImplementedError

    def make_host(self):
        raise NotImplementedError

    takes_mapping = True

    def setup(self, torch, lib, stream):
        import cubutterfly_amd as cb
        self.plans = [cb.Plan(lib, self.transform(cb), options=self.plan_options(cb), stream=stream)]
        ws_bytes = self.plans[0].workspace_size()
        if ws_bytes:
            self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
            self.plans[0].set_workspace(self.workspace, ws_bytes)
        self.host = self.make_host()
        src = _np_to_torch(torch, self.host).to("cuda")
        sets = self._rotation(torch, self.bytes_per_call)
        self.inputs = [src.clone() for _ in range(sets)]
        self.outputs = [torch.empty_like(src) for _ in range(sets)]

    def call(self, index):
        k = index % len(self.inputs)
        self.plans[0].execute(self.inputs[k], self.outputs[k])

    def timed_cpu(self, fn, what):
        reps, elapsed = 0, 0.0
        while elapsed < 10.0:
            t0 = time.perf_counter()
            fn()
            elapsed += time.perf_counter() - t0
            reps += 1
        return elapsed, reps * self.transforms_per_call, f"{reps} full batches ({what})"


class FftC64(OnePlan):
    """C3: complex64 FFT forward, 1 x 2^24 (c3a) or 1024 x 2^14 (c3b)."""
    dtype = "c64"

    def __init__(self, log_n, batch):
        self.log_n, self.batch = log_n, batch
        self.name = "c3a" if batch == 1 else "c3b"
        self.description = f"complex FFT c64 forward, batch {batch} x n=2^{log_n}, N(0,1) real and imaginary parts"
        self.transforms_per_call = batch
        self.bytes_per_call = 2 * batch * (8 << log_n)

    def transform(self, cb):
        return cb.Transform(op=cb.Operator.FFT, storage=cb.DataType.COMPLEX_FP32, compute=cb.ComputeType.FP32,
                            extents=[1 << self.log_n], batch=self.batch)

    def make_host(self):
        from cubutterfly_amd import workloads
        return workloads.complex_input(self.log_n, self.batch, seed=3).reshape(self.batch, 1 << self.log_n)

    def verify(self, torch):
        got = self.outputs[0].cpu().numpy().astype(np.complex128)
        ref = np.fft.fft(self.host.astype(np.complex128), axis=-1)
        err = np.linalg.norm(got - ref, axis=-1) / np.linalg.norm(ref, axis=-1)
        return bool(np.max(err) <= 1e-5)

    def cpu_sample(self, threads):
        import oracle
        return self.timed_cpu(lambda: oracle.fft_c64(self.host, threads=threads),
                              f"{self.batch} x 2^{self.log_n} through reference_fft, iterative radix-2")


class FftC64Rank2(FftC64):
    """Rank-2 complex64 FFT, 4096 x 4096 (not a BASELINE line): the composite
    plan (row transforms, tiled transposes, column transforms)."""

    def __init__(self):
        super().__init__(24, 1)
        self.name = "r2"
        self.description = "rank-2 complex FFT c64 forward, 4096 x 4096, batch 1, N(0,1) parts"

    def transform(self, cb):
        return cb.Transform(op=cb.Operator.FFT, storage=cb.DataType.COMPLEX_FP32, compute=cb.ComputeType.FP32,
                            extents=[4096, 4096], batch=1)

    def verify(self, torch):
        got = self.outputs[0].cpu().numpy().reshape(4096, 4096).astype(np.complex128)
        ref = np.fft.fft2(self.host.reshape(4096, 4096).astype(np.complex128))
        return bool(np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5)

    def cpu_sample(self, threads):
        import oracle

        def both_axes():
            rows = oracle.fft_c64(self.host.reshape(4096, 4096), threads=threads)
            oracle.fft_c64(np.ascontiguousarray(rows.T), threads=threads)

        return self.timed_cpu(both_axes, "4096 x 4096 through reference_fft along both axes")


class FwhtFp16(OnePlan):
    """C5: QuaRot-style FP16 FWHT, scale 1/sqrt(n), FP32 compute, one final
    FP16 rounding: 16384 x 4096 (c5a) or 524288 x 128 (c5b)."""
    dtype = "f16"

    def __init__(self, rows, n):
        self.rows, self.n = rows, n
        self.name = "c5a" if n == 4096 else "c5b"
        self.description = (f"FWHT fp16 storage / fp32 compute, {rows} x n={n}, output scale 1/sqrt(n), "
                            "final-storage rounding, activations with outlier channels")
        self.transforms_per_call = rows
        self.bytes_per_call = 2 * rows * n * 2
        self.scale = float(np.float32(1.0 / np.sqrt(n)))

    def transform(self, cb):
        return cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP16, compute=cb.ComputeType.FP32,
                            extents=[self.n], batch=self.rows, output_scale=self.scale,
                            output_rounding=cb.OutputRounding.FINAL_STORAGE)

    def make_host(self):
        from cubutterfly_amd import workloads
        return workloads.quarot_input(self.rows, self.n, seed=5)

    def verify(self, torch):
        import oracle
        got = self.outputs[0].cpu().numpy().view(np.float16).astype(np.float32)
        ref = oracle.fwht_f16_final(self.host, self.scale, threads=oracle.default_threads()).astype(np.float32)
        return bool(np.max(np.abs(got - ref)) <= 2e-3)

    def cpu_sample(self, threads):
        import oracle
        return self.timed_cpu(lambda: oracle.fwht_f16_final(self.host, self.scale, threads=threads),
                              f"{self.rows} x {self.n} through reference_fwht in fp32 + one fp16 rounding")


class DeviceCopy(Workload):
    """Calibration probe, not a BASELINE config: a plain device-to-device copy
    of 128 MiB, the known-size reference for rocprofv3 FETCH_SIZE/WRITE_SIZE."""
    name = "copy"
    dtype = "u8"
    description = "plain device copy of 134217728 bytes (HBM traffic counter calibration)"
    transforms_per_call = 1
    bytes_per_call = 2 * 134217728

    def setup(self, torch, lib, stream):
        sets = self._rotation(torch, self.bytes_per_call)
        self.inputs = [torch.ones(134217728 // 4, dtype=torch.float32, device="cuda") for _ in range(sets)]
        self.outputs = [torch.empty_like(self.inputs[0]) for _ in range(sets)]

    def call(self, index):
        k = index % len(self.inputs)
        self.outputs[k].copy_(self.inputs[k])

    def kernel_name(self):
        return "torch copy_"

    def cpu_sample(self, threads):
        return 1.0, 0, "no CPU baseline for the calibration copy"


WORKLOADS = {"c1": FwhtFp32, "c1p": FwhtFp32Pitched, "c2": NttNegacyclic, "c3a": lambda: FftC64(24, 1), "c3b": lambda: FftC64(14, 1024),
             "c4": RnsNegacyclic, "c5a": lambda: FwhtFp16(16384, 4096), "c5b": lambda: FwhtFp16(524288, 128),
             "r2": FftC64Rank2, "copy": DeviceCopy}
DEFAULT_WORKLOAD = "c2"


CALLS_PER_GRAPH = 20
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic.txt")


def measured_traffic(name):
    """HBM bytes per call (read + write) for a workload, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE summary in profiles/ (scaled by the copy-kernel
    calibration recorded there), or None when no measurement exists."""
    try:
        with open(TRAFFIC_TABLE) as f:
            for line in f:
                fields = line.split()
                if len(fields) == 3 and fields[0] == name:
                    return int(fields[1]) + int(fields[2])
    except OSError:
        pass
    return None


def time_calls(torch, workload, stream, steps, warmup, use_graph=True):
    """Milliseconds per call. W eager warmup calls; then, as the reference
    times it (a graph of 20 calls replayed, docs/fwht_native_repair_20261107.md:20),
    the K timed calls run as replays of a captured HIP graph of 20 calls so
    host submission is not measured. Events are recorded on the plans' stream."""
    with torch.cuda.stream(stream):
        for i in range(warmup):
            workload.call(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(CALLS_PER_GRAPH):
                workload.call(i)
        torch.cuda.synchronize()
        replays = max(1, -(-steps // CALLS_PER_GRAPH))
        # replay() launches on the current stream: make it the plans' stream.
        with torch.cuda.stream(stream):
            graph.replay()  # first replay uploads the graph
            torch.cuda.synchronize()
            start.record(stream)
            for _ in range(replays):
                graph.replay()
            stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / (replays * CALLS_PER_GRAPH), replays * CALLS_PER_GRAPH
    start.record(stream)
    with torch.cuda.stream(stream):
        for i in range(steps):
            workload.call(warmup + i)
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps, steps


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--verify", action="store_true", help="check one output against the oracle")
    parser.add_argument("--eager", action="store_true", help="time eager submissions instead of graph replays")
    parser.add_argument("--mapping", default=None,
                        help="plan one-plan workloads with this lowering (EXPLICIT policy) instead of the default")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the butterfly path is single-GPU (every configuration "
              "shards by rows/limbs with no communication); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import cubutterfly_amd as cb
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    lib = cb.Library()
    stream = torch.cuda.Stream()  # default priority; plans launch on it
    workload = WORKLOADS[args.workload]()
    if args.mapping:
        if not workload.takes_mapping:
            print(f"--mapping applies to one-plan workloads; {args.workload} is not one", file=sys.stderr)
            sys.exit(2)
        workload.mapping = args.mapping
    workload.setup(torch, lib, stream.cuda_stream)
    torch.cuda.synchronize()

    ms, timed = time_calls(torch, workload, stream, args.steps, args.warmup, use_graph=not args.eager)
    transforms_per_s = workload.transforms_per_call / (ms * 1e-3)
    achieved = workload.bytes_per_call / (ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": transforms_per_s,
        "unit": "transforms/s",
        "n_gpus": 1,
        "steps": timed,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": workload.dtype,
        "data": "synthetic (seeded splitmix64 / mt19937_64 generators)",
        "config": workload.config(),
        "roofline": {
            "bound": "hbm",
            "kernel": workload.kernel_name(),
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(workload.name),
            "algorithmic_bytes_per_call": workload.bytes_per_call,
        },
        "timing": "hip graph of %d calls, replayed" % CALLS_PER_GRAPH if not args.eager else "eager calls",
    }
    if hasattr(workload, "valu_per_butterfly"):
        # The integer-VALU roof of the NTT configs (see VALU_LANE_OPS_PER_S).
        rate = workload.butterflies_per_call / (ms * 1e-3)
        peak = VALU_LANE_OPS_PER_S / workload.valu_per_butterfly
        result["valu_roofline"] = {
            "bound": "valu",
            "achieved": rate,
            "peak": peak,
            "unit": "butterflies/s",
            "frac": rate / peak,
            "valu_per_butterfly": workload.valu_per_butterfly,
            "floor_ms_per_step": workload.butterflies_per_call / peak * 1e3,
        }
    if args.verify:
        result["verified"] = workload.verify(torch)
    if not args.no_cpu:
        import oracle
        threads = oracle.default_threads()
        seconds, transforms, sample = workload.cpu_sample(threads)
        result["cpu_baseline"] = {
            "value": transforms / seconds,
            "unit": "transforms/s",
            "cores": threads,
            "kind": "port",
            "sample": sample + f"; {seconds:.1f} s on {threads} host threads",
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
