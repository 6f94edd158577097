"""MI355X-native paged K/V-cache hot path for cache-aware FastConformer streaming.

Drop-in host modules mirror the reference package layout:

* ``parakeet_amd.modules.cache``      -- ``ModelCache``, ``StreamingState`` (paged)
* ``parakeet_amd.modules.attention``  -- ``PositionalEncoding``, ``ConformerAttention``
* ``parakeet_amd.modules.encoder``    -- ``ConformerEncoder`` (streaming state, masks, layer loop)
* ``parakeet_amd.engine.scheduler``   -- ``Scheduler`` (slot pool + paged batches)

``parakeet_amd.ops`` exposes the kernels; ``parakeet_amd.pool`` the host page pool.
"""

from . import ops, pool
from ._lib import LIB_PATH, lib

__all__ = ["ops", "pool", "lib", "LIB_PATH"]
