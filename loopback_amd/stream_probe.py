"""The practical streaming ceilings of the box for the read kernels' access patterns (libloopback_probe.so):

  * read-only, 32 sources of 64 MiB streamed row by row (the read kernels' pattern, nothing written);
  * the same with one 4 KiB row written per row set (1 write per 32 reads, the read forward's mix), each row right
    after its reads, or 16 consecutive rows kept in LDS and written together (the read forward's staged output);
  * the write step's traffic, two rows in and one out per token (16384 x 2048 bf16), in the write kernel's chunked
    layout (128 bytes of a row per lane group) and in whole rows per wave;
  * a device copy (1 read, 1 write per element);
each at several grid sizes, best of 5. Reported as GB/s of the bytes each probe moves, beside the 8 TB/s peak.

    python -m loopback_amd.stream_probe        # one JSON line + a table
"""
from __future__ import annotations

import ctypes
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "libloopback_probe.so")
PEAK_GBS = 8000.0


def _lib():
    if not os.path.exists(PATH):
        raise ImportError(f"{PATH} is not built (python -m loopback_amd.build)")
    lib = ctypes.CDLL(PATH)
    lib.ldp_read.restype = ctypes.c_int
    lib.ldp_read.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_int, ctypes.c_int64, ctypes.c_void_p,
                             ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.ldp_read_burst.restype = ctypes.c_int
    lib.ldp_read_burst.argtypes = lib.ldp_read.argtypes
    lib.ldp_write.restype = ctypes.c_int
    lib.ldp_write.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                              ctypes.c_void_p]
    lib.ldp_copy.restype = ctypes.c_int
    lib.ldp_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    return lib


def _best(fn, reps=5):
    best = float("inf")
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e-3)
    return best


def main():
    if not torch.cuda.is_available():
        print("stream_probe: no GPU visible", file=sys.stderr)
        sys.exit(3)
    lib = _lib()
    dev = torch.device("cuda", 0)
    n, rows = 32, 16384                                   # 32 sources x 16384 rows x 4 KiB = 2 GiB
    gen = torch.Generator(device=dev).manual_seed(0)
    src = torch.randint(0, 1 << 30, (n, rows * 1024), dtype=torch.int32, device=dev, generator=gen)
    out = torch.empty(rows * 1024, dtype=torch.int32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    ptrs = (ctypes.c_uint64 * n)(*[src[i].data_ptr() for i in range(n)])
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    row_bytes, src_bytes = 4096, n * rows * 4096

    def check(code, what):
        if code != 0:
            raise RuntimeError(f"stream_probe: {what} failed ({code})")

    res = {}
    for grid in (512, 1024, 2048, 4096):
        ro = _best(lambda: check(lib.ldp_read(ptrs, n, rows, None, ctypes.c_void_p(sink.data_ptr()), grid, st),
                                 "read"))
        rw = _best(lambda: check(lib.ldp_read(ptrs, n, rows, ctypes.c_void_p(out.data_ptr()),
                                              ctypes.c_void_p(sink.data_ptr()), grid, st), "read+write"))
        rb = _best(lambda: check(lib.ldp_read_burst(ptrs, n, rows, ctypes.c_void_p(out.data_ptr()),
                                                    ctypes.c_void_p(sink.data_ptr()), grid, st), "read+burst write"))
        cp = _best(lambda: check(lib.ldp_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(src[n // 2].data_ptr()),
                                              src_bytes // 2, grid, st), "copy"))
        res[grid] = {"read_32_sources": src_bytes / ro / 1e9,
                     "read_32_sources_write_1": (src_bytes + rows * row_bytes) / rw / 1e9,
                     "read_32_sources_write_1_burst16": (src_bytes + rows * row_bytes) / rb / 1e9,
                     "copy": src_bytes / cp / 1e9}
    best = {k: max(r[k] for r in res.values()) for k in next(iter(res.values()))}
    # the write step's traffic (h, x in; v out; 16384 rows of 2048 bf16), its own grid of 64-token workgroups
    wrows = 16384
    hw = src[0].view(torch.bfloat16)[: wrows * 2048]
    xw = src[1].view(torch.bfloat16)[: wrows * 2048]
    vw = out.view(torch.bfloat16)[: wrows * 2048]   # out holds exactly 16384 x 2048 bf16
    for which, key in ((0, "write_h_x_chunked"), (1, "write_h_x_rows")):
        t = _best(lambda: check(lib.ldp_write(ctypes.c_void_p(hw.data_ptr()), ctypes.c_void_p(xw.data_ptr()),
                                              ctypes.c_void_p(vw.data_ptr()), wrows, which, st), key))
        best[key] = 3 * wrows * 2048 * 2 / t / 1e9
    print(json.dumps({"metric": "streaming ceilings (GB/s of bytes moved)", "peak_gbs": PEAK_GBS, "best": best,
                      "by_grid": {str(g): r for g, r in res.items()}}), flush=True)
    print("| probe | best GB/s | of peak |")
    print("|---|---|---|")
    for k, v in best.items():
        print(f"| {k} | {v:.0f} | {v / PEAK_GBS:.2f} |")


if __name__ == "__main__":
    main()
