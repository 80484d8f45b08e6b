"""Calibration run for the HBM byte counters.

Copies 1 GiB three times with the bench-kit streaming copy kernel (one 16-byte
load and store per element), so rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this
run give the counters' reading for a known 1 GiB read + 1 GiB write:

    rocprofv3 --pmc FETCH_SIZE -- python3 friday-inference-engine_amd/hbm_calib.py
"""
import ctypes as C
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import friday_attn as fa  # noqa: E402


def main():
    fa.load()
    bk = C.CDLL(os.path.join(HERE, "lib", "libfa_benchkit.so"))
    bk.fabk_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
    n = 1 << 30
    a, b = fa.DeviceBuffer(n), fa.DeviceBuffer(n)
    for _ in range(3):
        bk.fabk_copy(a.ptr, b.ptr, n, None)
    fa.Hip.sync()
    print(f"copied {n} bytes x3")


if __name__ == "__main__":
    main()
