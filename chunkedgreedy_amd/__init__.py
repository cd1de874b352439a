"""chunkedgreedy_amd -- MI355X-native Chunked Greedy reordering + CSR SpMM.

Layout:
  csrc/        HIP kernels for gfx950 and the C ABI (include/sporder.h)
  build.py     in-tree hipcc build of libsporder_hip.so
  _lib.py      ctypes signatures of the C ABI
  sporder/     the reference's Python API (drop-in)
  synth.py     seeded synthetic CSR generators for the benchmark configs
  harness.py   counterparts of the reference's bench plugins (reorder method,
               SpMMMethod, cache flush)
"""

from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsporder_hip.so"

__all__ = ["LIB_PATH"]
