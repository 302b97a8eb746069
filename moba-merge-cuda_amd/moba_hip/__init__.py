"""moba_hip: MI355X-native (gfx950) MoBA sparse block attention.

Importing the package registers the ``opt_hip`` (GQA/MQA/MHA) and
``opt_merge_hip`` (MHA contract) prefill entries in :mod:`moba_hip.api`,
mirroring src/moba_opt/__init__.py:3-7, and exports the decode caches.
"""
from . import baseline_adapter  # noqa: F401
from . import grouped_attention  # noqa: F401  (registers opt_hip, opt_merge_hip)
from .api import available_impls, register, run_impl  # noqa: F401
from .grouped_attention import opt_hip, opt_hip_mha  # noqa: F401
from .merge import merge_forward  # noqa: F401
from .kv_cache import ContiguousKVCache, DecodeResult, PagedKVCache  # noqa: F401
from .prepared_decode import PreparedDecode  # noqa: F401
