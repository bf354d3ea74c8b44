#!/usr/bin/env python3
"""HBM calibration for the paged FP8 decode library on MI355X.

Runs the library's plain streaming kernels on buffers of a known size:

* ``l20_pd_stream_read``  -- reads ``--bytes`` once per launch (the read ceiling);
* ``l20_pd_stream_copy``  -- reads and writes ``--bytes`` once per launch;
* ``--launch-floor``      -- the time per launch of a near-empty kernel, issued
  back to back from the host and replayed from a HIP graph.

Rotating ``--buffers`` buffers keeps every launch cold in the 256 MB MALL.
Prints one JSON line with the measured rates.  Under ``rocprofv3 --pmc
FETCH_SIZE`` (or ``WRITE_SIZE``) the copy launches give the counter reading
for a known byte count, which scales the same counter read on the attention
kernels into HBM bytes.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
if str(HERE) not in sys.path:
    sys.path.insert(0, str(HERE))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--bytes", type=int, default=2**30)
    ap.add_argument("--buffers", type=int, default=3)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--blocks", type=int, default=4096)
    ap.add_argument("--launch-floor", action="store_true",
                    help="also time near-empty launches, eager and from a HIP graph")
    args = ap.parse_args()

    import torch

    import l20_pd_cabi as cabi

    assert torch.cuda.is_available(), "needs an MI355X"
    lib = cabi.load()
    n = args.bytes // 16 * 16
    src = [torch.ones(n, dtype=torch.uint8, device="cuda") for _ in range(args.buffers)]
    dst = [torch.empty(n, dtype=torch.uint8, device="cuda") for _ in range(args.buffers)]
    sink = torch.zeros(65536, dtype=torch.int32, device="cuda")
    h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def read(i):
        rc = lib.l20_pd_stream_read(ctypes.c_void_p(src[i].data_ptr()), ctypes.c_int64(n),
                                    ctypes.c_void_p(sink.data_ptr()), args.blocks, h)
        assert rc == 0, lib.l20_pd_last_error()

    def copy(i):
        rc = lib.l20_pd_stream_copy(ctypes.c_void_p(src[i].data_ptr()), ctypes.c_void_p(dst[i].data_ptr()),
                                    ctypes.c_int64(n), args.blocks, h)
        assert rc == 0, lib.l20_pd_last_error()

    out = {"bytes": n, "buffers": args.buffers, "steps": args.steps, "blocks": args.blocks,
           "device": getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")}
    for name, fn, moved in (("stream_read", read, n), ("stream_copy", copy, 2 * n)):
        for i in range(args.buffers):
            fn(i)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        for k in range(args.steps):
            ev[k][0].record()
            fn(k % args.buffers)
            ev[k][1].record()
        torch.cuda.synchronize()
        us = statistics.median(a.elapsed_time(b) * 1e3 for a, b in ev)
        out[name] = {"us_median": round(us, 2), "GBs": round(moved / us / 1e3, 1)}
    if args.launch_floor:
        out["launch_floor"] = launch_floor(lib, sink)
    print(json.dumps(out), flush=True)


def launch_floor(lib, sink, launches: int = 400):
    """Time per launch of a near-empty kernel (``l20_pd_stream_read`` of 16 bytes),
    issued back to back from the host and replayed from a captured HIP graph.
    The eager figure includes the host's per-launch cost (ctypes and
    hipLaunchKernel), the graph figure only the device's dispatch and drain."""
    import torch

    tiny = torch.ones(16, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    h = ctypes.c_void_p(side.cuda_stream)
    res = {}
    with torch.cuda.stream(side):
        for blocks in (1, 256, 1024):
            def one():
                rc = lib.l20_pd_stream_read(ctypes.c_void_p(tiny.data_ptr()), ctypes.c_int64(16),
                                            ctypes.c_void_p(sink.data_ptr()), blocks, h)
                assert rc == 0, lib.l20_pd_last_error()

            for _ in range(20):
                one()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(side)
            for _ in range(launches):
                one()
            e.record(side)
            torch.cuda.synchronize()
            eager = s.elapsed_time(e) * 1e3 / launches
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(launches):
                    one()
            graph.replay()
            torch.cuda.synchronize()
            s.record(side)
            graph.replay()
            e.record(side)
            torch.cuda.synchronize()
            res[f"{blocks}_workgroups"] = {"eager_us": round(eager, 2),
                                           "graph_us": round(s.elapsed_time(e) * 1e3 / launches, 2)}
    return res


if __name__ == "__main__":
    main()
