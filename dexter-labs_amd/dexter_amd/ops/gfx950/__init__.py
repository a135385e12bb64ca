"""HIP kernels for AMD CDNA4 (gfx950, Instinct MI355X).

What shapes these kernels, as against dexter's RDNA3.5 Triton set
(``python/dexter/ops/gfx1151/__init__.py``):

* **wave64 + MFMA.** Products run on ``v_mfma_f32_32x32x16_{bf16,f16}``: a
  32x32 fp32 accumulator over 64 lanes. Attention computes S^T = K Q^T so a
  lane owns one query and the softmax statistics need no cross-lane traffic
  beyond one exchange per tile.
* **160 KB LDS per CU, 256 CUs in 8 XCDs.** K and V^T tiles are staged in LDS;
  decode-shaped calls split the key range over workgroups so all CUs stream
  the cache; all workgroups of one head are placed on one XCD (one L2).
* **HBM3E at 8 TB/s.** The 83-token decode chunk is bandwidth-bound: the
  cache is read once, in place, with no concatenation copy.

All kernels live in one shared library with a C ABI
(``include/dexter_gfx950.h``), loaded with ctypes by ``_lib``. Importing this
package registers the implementations; it does not load the library, so
registration works on any machine and only a call on a gfx950 needs it.
"""

from . import attention, cache, fused, norm, proj, rope  # noqa: F401
