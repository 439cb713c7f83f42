"""Per-op throughput of the decode kernels at the BASELINE op configs (1-4),
and of the prefill NF4 GEMMs at 64 tokens (6).

    python -m kudacuda_amd.opbench [--configs 1 2 3 4 6] [--launches 256]

Each measurement captures ``launches`` back-to-back calls of one C-ABI entry
point into a hipGraph (so host launch cost is excluded), cycling through
enough distinct copies of the weights (or KV caches) that the working set
exceeds 512 MiB -- twice the MI355X's 256 MiB last-level cache -- so every
launch streams its bytes from HBM.  One JSON line per case:
``{op, config, us, bytes, gbs, frac}`` with bytes the algorithmic HBM bytes
of one launch and frac = GB/s / 8000.  Inputs are seeded synthetic tensors
of the config's shape; values do not affect timing.
"""

from __future__ import annotations

import argparse
import json
import math
import sys
from typing import Any, Callable

import numpy as np

PEAK_GBS = 8000.0
WORKING_SET = 512 << 20
GQA_LENGTHS = (1, 7, 128, 512, 585, 1024, 2048, 8192, 32768)


def _nf4_bytes(rows: int, cols: int) -> int:
    return rows * cols // 2 + rows * cols // 64 * 4


class Bench:
    def __init__(self, torch: Any, launches: int) -> None:
        from ._native import Native

        self.torch = torch
        self.native = Native(0)
        self.stream = torch.cuda.Stream()
        self.launches = launches
        self.dev = "cuda:0"
        self.results: list[dict[str, Any]] = []
        self.echo = True

    def copies_for(self, nbytes: int) -> int:
        return max(1, min(self.launches, math.ceil(WORKING_SET / max(nbytes, 1))))

    def rand_u8(self, n: int) -> Any:
        return self.torch.randint(0, 256, (n,), dtype=self.torch.uint8, device=self.dev)

    def rand_bf16(self, n: int, std: float = 1.0) -> Any:
        return (self.torch.randn(n, device=self.dev) * std).to(self.torch.bfloat16)

    def absmax(self, n: int) -> Any:
        return self.torch.rand(n, device=self.dev) * 0.05 + 0.01

    def time(self, launch: Callable[[int], None]) -> float:
        """Mean microseconds per launch of a captured sequence (launch(i) issues call i)."""

        lib, handle, s = self.native.lib, self.native.handle, self.stream.cuda_stream
        self.torch.cuda.synchronize()
        self.native.check(lib.kudacuda_reset_graph(handle), "kudacuda_reset_graph")
        self.native.check(lib.kudacuda_begin_capture(handle, s), "kudacuda_begin_capture")
        for i in range(self.launches):
            launch(i)
        self.native.check(lib.kudacuda_end_capture(handle, s), "kudacuda_end_capture")
        for _ in range(2):
            self.native.check(lib.kudacuda_replay_graph(handle, s), "kudacuda_replay_graph")
        start = self.torch.cuda.Event(enable_timing=True)
        stop = self.torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        self.native.check(lib.kudacuda_replay_graph(handle, s), "kudacuda_replay_graph")
        stop.record(self.stream)
        stop.synchronize()
        return start.elapsed_time(stop) * 1e3 / self.launches

    def report(self, op: str, config: int, us: float, nbytes: int, **extra: Any) -> None:
        gbs = nbytes / (us * 1e-6) / 1e9
        line = {"op": op, "config": config, "us": round(us, 3), "bytes": nbytes, "gbs": round(gbs, 1),
                "frac": round(gbs / PEAK_GBS, 4)}
        line.update(extra)
        self.results.append(line)
        if self.echo:
            print(json.dumps(line), flush=True)

    # ---------------------------------------------------------------- configs
    def gemv(self) -> None:
        nbytes = _nf4_bytes(2048, 2048) + 2 * 2048 * 2
        n = self.copies_for(nbytes)
        w = [self.rand_u8(2048 * 1024) for _ in range(n)]
        a = [self.absmax(2048 * 32) for _ in range(n)]
        x, y = self.rand_bf16(2048), self.rand_bf16(2048)
        s = self.stream.cuda_stream

        def launch(i: int) -> None:
            self.native.call("kudacuda_nf4_gemv_bf16", x.data_ptr(), w[i % n].data_ptr(), a[i % n].data_ptr(), 0, 0,
                             y.data_ptr(), 1, 2048, 2048, 64, s)

        self.report("nf4_gemv_2048x2048", 1, self.time(launch), nbytes, copies=n)

    def qkv(self) -> None:
        nbytes = _nf4_bytes(2560, 2048) + 2 * 2560 + 2 * 2048 * 2 + 2 * 2560
        n = self.copies_for(nbytes)
        ws = [[(self.rand_u8(r * 1024), self.absmax(r * 32)) for r in (2048, 256, 256)] for _ in range(n)]
        bias = [self.rand_bf16(r, 0.01) for r in (2048, 256, 256)]
        x, g = self.rand_bf16(2048), self.rand_bf16(2048, 0.1) + 1
        outs = [self.rand_bf16(r) for r in (2048, 256, 256)]
        s = self.stream.cuda_stream

        def launch(i: int) -> None:
            (qw, qa), (kw, ka), (vw, va) = ws[i % n]
            self.native.call("kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16", x.data_ptr(), g.data_ptr(),
                             qw.data_ptr(), qa.data_ptr(), bias[0].data_ptr(), kw.data_ptr(), ka.data_ptr(),
                             bias[1].data_ptr(), vw.data_ptr(), va.data_ptr(), bias[2].data_ptr(),
                             outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), 1, 2048, 2048, 256, 64,
                             1e-6, s)

        self.report("fused_rmsnorm_qkv_nf4", 2, self.time(launch), nbytes, copies=n)

    def mlp(self) -> None:
        gate_up = 2 * _nf4_bytes(11008, 2048) + 2 * 2048 * 2 + 2 * 11008
        down = _nf4_bytes(2048, 11008) + 2 * 11008 + 2 * 2048 * 2
        nbytes = gate_up + down
        n = self.copies_for(nbytes)
        gu = [[(self.rand_u8(11008 * 1024), self.absmax(11008 * 32)) for _ in range(2)] for _ in range(n)]
        dn = [(self.rand_u8(2048 * 5504), self.absmax(2048 * 172)) for _ in range(n)]
        x, g = self.rand_bf16(2048), self.rand_bf16(2048, 0.1) + 1
        h, y = self.rand_bf16(11008), self.rand_bf16(2048)
        s = self.stream.cuda_stream

        def launch_mlp(i: int) -> None:
            (gw, ga), (uw, ua) = gu[i % n]
            dw, da = dn[i % n]
            self.native.call("kudacuda_qwen2_mlp_nf4_bf16", x.data_ptr(), g.data_ptr(), gw.data_ptr(),
                             ga.data_ptr(), uw.data_ptr(), ua.data_ptr(), dw.data_ptr(), da.data_ptr(),
                             h.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 2048, 11008, 64, 1e-6, s)

        def launch_swiglu(i: int) -> None:
            (gw, ga), (uw, ua) = gu[i % n]
            self.native.call("kudacuda_qwen2_swiglu_nf4_bf16", x.data_ptr(), g.data_ptr(), gw.data_ptr(),
                             ga.data_ptr(), uw.data_ptr(), ua.data_ptr(), h.data_ptr(), 1, 2048, 11008, 64, 1e-6, s)

        self.report("mlp_nf4_gate_up_down", 3, self.time(launch_mlp), nbytes, copies=n)
        self.report("swiglu_nf4_gate_up", 3, self.time(launch_swiglu), gate_up, copies=n)

    def prefill_gemm(self) -> None:
        """NF4 GEMMs of the multi-token prefill at M = 64 tokens (MFMA): bytes =
        NF4 weights + absmax + bf16 activations in and out; flops = 2 M N K."""

        m = 64
        s = self.stream.cuda_stream
        cases = (("q_proj", 2048, 2048, False), ("gate_up_swiglu", 11008, 2048, True), ("down", 2048, 11008, False))
        for name, n, k, swiglu in cases:
            nw = 2 if swiglu else 1
            nbytes = nw * _nf4_bytes(n, k) + 2 * m * k + 2 * m * n
            copies = self.copies_for(nbytes)
            ws = [[(self.rand_u8(n * k // 2), self.absmax(n * k // 64)) for _ in range(nw)] for _ in range(copies)]
            x, y = self.rand_bf16(m * k), self.rand_bf16(m * n)

            def launch(i: int, ws=ws, x=x, y=y, n=n, k=k, swiglu=swiglu) -> None:
                w = ws[i % len(ws)]
                if swiglu:
                    self.native.call("kudacuda_nf4_gemm_swiglu_bf16", x.data_ptr(), w[0][0].data_ptr(),
                                     w[0][1].data_ptr(), w[1][0].data_ptr(), w[1][1].data_ptr(), y.data_ptr(), m, k,
                                     n, 64, s)
                else:
                    self.native.call("kudacuda_nf4_gemm_bf16", x.data_ptr(), w[0][0].data_ptr(), w[0][1].data_ptr(),
                                     0, 0, y.data_ptr(), m, k, n, 64, s)

            us = self.time(launch)
            self.report(f"prefill_gemm_{name}", 6, us, nbytes, tokens=m, copies=copies,
                        tflops=round(2.0 * m * n * k * nw / (us * 1e-6) / 1e12, 2))
            del ws
            self.torch.cuda.empty_cache()

    def gqa(self, lengths: tuple[int, ...] = GQA_LENGTHS) -> None:
        s = self.stream.cuda_stream
        scale = 1.0 / math.sqrt(128.0)
        for length in lengths:
            nbytes = 1024 * length + 8192
            n = self.copies_for(nbytes)
            caches = [(self.rand_bf16(2 * length * 128), self.rand_bf16(2 * length * 128)) for _ in range(n)]
            q, out = self.rand_bf16(2048), self.rand_bf16(2048)

            def launch(i: int) -> None:
                k, v = caches[i % n]
                self.native.call("kudacuda_qwen2_gqa_decode_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                 out.data_ptr(), 1, 1, length, 16, 2, 128, scale, s)

            self.report("gqa_decode_bf16", 4, self.time(launch), nbytes, kv_len=length, copies=n)
            del caches
            self.torch.cuda.empty_cache()


def collect(torch: Any, configs: tuple[int, ...] = (1, 2, 3, 4), launches: int = 128) -> list[dict[str, Any]]:
    """Measure ``configs`` and return one result dict per case (no printing)."""

    bench = Bench(torch, launches)
    bench.echo = False
    try:
        with torch.cuda.stream(bench.stream):
            for config in configs:
                {1: bench.gemv, 2: bench.qkv, 3: bench.mlp, 4: bench.gqa, 6: bench.prefill_gemm}[config]()
                torch.cuda.empty_cache()
    finally:
        bench.native.close()
    return bench.results


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--configs", type=int, nargs="+", default=[1, 2, 3, 4, 6])
    parser.add_argument("--launches", type=int, default=256)
    parser.add_argument("--copy-mib", type=int, default=0,
                        help="first run 3 plain device copies of this many MiB (counter calibration)")
    parser.add_argument("--gqa-lengths", type=int, nargs="+", default=list(GQA_LENGTHS),
                        help="kv lengths of config 4")
    args = parser.parse_args(argv)
    import torch

    torch.manual_seed(20260824)
    bench = Bench(torch, args.launches)
    with torch.cuda.stream(bench.stream):
        if args.copy_mib > 0:
            src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=bench.dev).fill_(1)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            print(json.dumps({"op": "copy_calibration", "bytes_read": src.numel(), "bytes_written": dst.numel()}),
                  flush=True)
            del src, dst
        for config in args.configs:
            if config == 4:
                bench.gqa(tuple(args.gqa_lengths))
            else:
                {1: bench.gemv, 2: bench.qkv, 3: bench.mlp, 6: bench.prefill_gemm}[config]()
    bench.native.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
