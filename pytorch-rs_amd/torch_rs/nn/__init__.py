"""torch_rs.nn (hot-path subset: functional.relu and functional.dropout)."""
from . import functional  # noqa: F401
