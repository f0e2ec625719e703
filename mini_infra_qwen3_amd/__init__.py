"""MI355X-native paged-KV data plane for mini-infra-qwen3.

Drop-in for the reference's paged path: ``core`` keeps the block-table control plane
(``FreeKVCacheBlockQueue``, ``KVCacheManager``), ``worker`` the ``PagedKVCachePool`` and
``PagedRunner`` entry points, ``model`` the Qwen3 attention whose paged branch calls the
HIP kernels of ``libmi_paged.so`` (``data_plane`` / ``_native``).  Dense GEMMs stay on
PyTorch-ROCm.
"""

__version__ = "0.1.0"
