"""Host-side layout driver of the paged KV cache (pure Python, no GPU work)."""
from .block_manager import Block, BlockManager  # noqa: F401
from .context import AttentionContext, get_context, reset_context, set_context  # noqa: F401
from .kv_manager import PagedKVManager  # noqa: F401
from .prefix_cache import PrefixCache  # noqa: F401
from .sequence import Sequence, SequenceStatus  # noqa: F401
