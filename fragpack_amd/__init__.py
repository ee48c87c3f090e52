"""FragPack on MI355X: lossless BF16 KV records and fused decode attention.

Host-side mirror of the reference package ``fragpack`` (compression and ops
layers) over hand-written gfx950 HIP kernels in ``libfragpack_hip.so``
(C ABI: include/fragpack_hip.h).
"""

__version__ = "0.1.0"
