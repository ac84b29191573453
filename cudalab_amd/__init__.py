"""cudalab_amd: MI355X (gfx950) weight-only quantized GEMV path.

W4A16 group-wise INT4 GEMV and W8A16 per-row INT8 GEMV as hand-written HIP
kernels behind a C ABI (include/cdnaqgemv.h, libcdnaqgemv.so), with the
reference's Python operator surface on top: `operators.get(name)`,
`build.build(op)` extension objects, the quantize/pack helpers, the
correctness and negative suites, and `dispatch`.
"""

__version__ = "0.1.0"
