"""Host-side layout driver of the paged KV cache.

Everything here is host logic, except ``DeviceBlockTables``, which keeps the block tables on the
GPU and derives each step's metadata there (it loads the library only when a step runs)."""
from .block_manager import Block, BlockManager  # noqa: F401
from .context import AttentionContext, get_context, reset_context, set_context  # noqa: F401
from .device_tables import DeviceBlockTables  # noqa: F401
from .kv_manager import PagedKVManager  # noqa: F401
from .prefix_cache import PrefixCache  # noqa: F401
from .sequence import Sequence, SequenceStatus  # noqa: F401
