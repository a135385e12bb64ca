"""dexter_amd: dexter's blockwise-causal attention path, native on MI355X (gfx950).

Layout mirrors the reference package ``python/dexter``:

* ``platform``  device description and capability gates (adds the CDNA4 row)
* ``registry``  priority/capability kernel registry, ``DEXTER_KERNEL`` pin
* ``ops``       ``qk_norm_rope``, ``blockwise_causal_attention``,
                ``kv_cache_append`` dispatchers
* ``ops.gfx950`` the HIP implementations behind a C-ABI shared library
* ``models``    ``KVCache`` and a ``SelfAttention``-style caller
"""

__version__ = "0.1.0"
