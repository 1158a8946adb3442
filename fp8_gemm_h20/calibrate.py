"""Calibration of the GPU this runs on: the FP8 MFMA rate (alone, and with the
block-scale promotion of every product) and the streaming read and write
rates it sustains, measured with the library's calibration kernels
(fp8bg_calib_mfma, fp8bg_calib_mfma_promoted, fp8bg_calib_read,
fp8bg_calib_write).  They are reported next to the
published peaks (5.0 PFLOP/s dense FP8, 8 TB/s HBM) that the roofline
fractions divide by, as the share of those peaks the chip itself reaches.
"""
import statistics

from . import _lib

MFMA_FLOPS = 2 * 16 * 16 * 128   # one FP8 16x16x128 MFMA
MFMA_PER_ITER = 16               # per wave and iteration (fp8bg_calib_mfma_kernel)
ONE_CODES = 0x38383838           # four e4m3 1.0 codes


def _num_cus(device):
    return _lib.num_cus(device.index if device.index is not None else 0)


def _time(torch, stream, launch, reps):
    launch()                                        # warm-up, untimed
    vals = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        launch()
        e1.record(stream)
        e1.synchronize()
        vals.append(e0.elapsed_time(e1) * 1e3)
    return statistics.median(vals)


def mfma_rate(torch, device, stream, iters=4096, workgroups_per_cu=2, reps=5, promoted=False):
    """Dense FP8 MFMA rate: workgroups_per_cu workgroups of 4 waves on every
    CU (two waves per SIMD by default, as the 256x256 GEMM tile runs), each
    wave issuing 16 MFMAs per iteration; with promoted, each product is
    promoted by four FMAs as in the GEMM kernels.  Checks every output
    (2048 * iters) and returns TFLOP/s."""
    lib = _lib.lib()
    wgs = _num_cus(device) * workgroups_per_cu
    codes = torch.full((32 * 64,), ONE_CODES, dtype=torch.int32, device=device)
    scale = torch.ones(64, dtype=torch.float32, device=device)
    out = torch.empty(wgs * 256, dtype=torch.float32, device=device)
    name = "fp8bg_calib_mfma_promoted" if promoted else "fp8bg_calib_mfma"
    stream.wait_stream(torch.cuda.current_stream(device))    # the fills above come first

    def launch():
        if promoted:
            _lib.check(lib.fp8bg_calib_mfma_promoted(codes.data_ptr(), scale.data_ptr(), out.data_ptr(),
                                                     wgs, iters, stream.cuda_stream))
        else:
            _lib.check(lib.fp8bg_calib_mfma(codes.data_ptr(), out.data_ptr(), wgs, iters,
                                            stream.cuda_stream))
    with torch.cuda.stream(stream):
        us = _time(torch, stream, launch, reps)
    torch.cuda.synchronize(device)
    if not bool((out == 2048.0 * iters).all()):
        raise RuntimeError(f"{name}: wrong result")
    flops = wgs * 4 * iters * MFMA_PER_ITER * MFMA_FLOPS
    return {"tflops": round(flops / us / 1e6, 1), "us": round(us, 1), "workgroups": wgs,
            "iters": iters}


def read_rate(torch, device, stream, nbytes=1 << 30, workgroups_per_cu=2, reps=5):
    """Streaming read rate of an nbytes buffer (larger than every cache by
    default), in GB/s.  Two workgroups per CU stream fastest on MI355X (6.3
    TB/s at 1 and 4 GiB); 4 to 32 per CU reach 4.6-5.5 TB/s."""
    lib = _lib.lib()
    wgs = _num_cus(device) * workgroups_per_cu
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=device)
    out = torch.empty(wgs * 256, dtype=torch.int32, device=device)
    stream.wait_stream(torch.cuda.current_stream(device))    # the fill above comes first

    def launch():
        _lib.check(lib.fp8bg_calib_read(buf.data_ptr(), buf.numel() * 4, out.data_ptr(), wgs,
                                        stream.cuda_stream))
    with torch.cuda.stream(stream):
        us = _time(torch, stream, launch, reps)
    torch.cuda.synchronize(device)
    return {"GBps": round(nbytes / us / 1e3, 1), "us": round(us, 1), "bytes": nbytes,
            "workgroups": wgs}


def write_rate(torch, device, stream, nbytes=1 << 30, workgroups_per_cu=2, reps=5, nontemporal=True):
    """Streaming write rate into an nbytes buffer, in GB/s: 16-byte stores,
    non-temporal by default as the GEMM kernels write C.  Checks that every
    word holds the written value."""
    lib = _lib.lib()
    wgs = _num_cus(device) * workgroups_per_cu
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=device)
    value = 0x3F803F80                               # two bf16 1.0
    stream.wait_stream(torch.cuda.current_stream(device))    # the zero fill comes first

    def launch():
        _lib.check(lib.fp8bg_calib_write(buf.data_ptr(), buf.numel() * 4, value, wgs,
                                         1 if nontemporal else 0, stream.cuda_stream))
    with torch.cuda.stream(stream):
        us = _time(torch, stream, launch, reps)
    torch.cuda.synchronize(device)
    if not bool((buf == value).all()):
        raise RuntimeError("fp8bg_calib_write: wrong contents")
    return {"GBps": round(nbytes / us / 1e3, 1), "us": round(us, 1), "bytes": nbytes,
            "workgroups": wgs, "nontemporal": bool(nontemporal)}
