"""CPU oracle for the quantized matvec/matmul path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The product
(mythos.cpp_amd / libmythos_oil.so) never calls it.

`Oracle` wraps liboracle.so (this repo's C restatement, oracle.c).
`Reference` wraps oracle/_ref/libref_*.so, the reference's own kernel sources
compiled in place by oracle/Makefile (present only where it was built);
`ReferenceModel` the reference's DenseModel (_ref/libref_model.so).
"""
from .bindings import Oracle, Reference, ReferenceModel, oracle_lib_path, ref_lib_path, build  # noqa: F401
