"""Re-export of the host tiers used by block streaming (the reference's core/tiered_store.py re-exports PinnedHost
from core/tiers/pinned.py)."""
from .tiers.pinned import PinnedHost, registered_bytes, release_all  # noqa: F401
