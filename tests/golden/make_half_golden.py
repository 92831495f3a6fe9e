"""Writes tests/golden/half_trunc.npz: known-answer vectors of the reference's boundary
conversion f32 -> f16 (include/infvino/Half.hpp:14-24, src/Half.cpp bulk path), produced by
the reference's own sources compiled into oracle/_ref/libref_half.so (make -C oracle).
The fixture lets the CPU tests pin the truncating conversion where the reference tree is
absent.  Inputs: special values (zeros, denormal boundaries, overflow boundaries, inf, nan)
and seeded random bit patterns."""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "..", "..", "oracle", "_ref", "libref_half.so")


def main():
    L = C.CDLL(LIB)
    L.ref_f32_to_f16_bulk.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 65536.0, 1e30, -1e30,
                        6.1035156e-05, 6.1e-05, 5.96e-08, 2.0 ** -14, 2.0 ** -15, 2.0 ** -24,
                        np.inf, -np.inf, np.nan, 0.1, 0.2, 1.0009765625, 1.00048828125, 3.14159],
                       np.float32)
    rng = np.random.default_rng(20261201)
    bits = rng.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32)
    normal = rng.normal(0, 100, 2000).astype(np.float32)
    x = np.concatenate([special, bits.view(np.float32), normal])
    h = np.empty(x.size, np.uint16)
    L.ref_f32_to_f16_bulk(x.ctypes.data, h.ctypes.data, x.size)
    np.savez_compressed(os.path.join(HERE, "half_trunc.npz"), x=x, h=h)
    print("wrote", x.size, "vectors")


if __name__ == "__main__":
    main()
