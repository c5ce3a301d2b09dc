"""Proves the sanitized libdsx.so build is live (CPU only, no GPU call):
dsx_build_chunks is told its output buffer holds 40 chunks when it holds 30
(720 bytes, so the buffer comes from malloc, which ASan guards), and writes
past the end. Under run.sh this must die with a heap-buffer-overflow report;
a clean exit means the instrumentation is missing."""
import ctypes
import sys

lib = ctypes.CDLL(sys.argv[1])
I64 = ctypes.c_int64
lib.dsx_build_chunks.restype = I64
lib.dsx_build_chunks.argtypes = [ctypes.c_void_p, ctypes.c_int32, I64, ctypes.c_void_p, I64]
numels = (I64 * 1)(40 * 8)
out = ctypes.create_string_buffer(30 * 24)
got = lib.dsx_build_chunks(numels, 1, 8, out, 40)
print(f"canary wrote {got} chunks without a report")
