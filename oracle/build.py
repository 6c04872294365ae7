"""Build the C restatement of the oracle (TEST INFRASTRUCTURE ONLY) into oracle/_build/liboracle.so with gcc."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build", "liboracle.so")


def build():
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-o", OUT, os.path.join(HERE, "e4m3.c"), "-lm"], check=True)
    return OUT


def load():
    import ctypes
    if not os.path.exists(OUT):
        build()
    L = ctypes.CDLL(OUT)
    L.oracle_e4m3_encode_bits.argtypes = [ctypes.c_uint32, ctypes.c_longlong, ctypes.c_void_p]
    L.oracle_e4m3_encode_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong]
    return L


if __name__ == "__main__":
    print(build())
