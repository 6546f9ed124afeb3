"""Reference names of the sparse decode entry points
(cvsa/kernels/sparse_decode.py:286, :537, :664, :681)."""
from ..ops import next_power_of_2 as _next_power_of_2  # noqa: F401
from ..ops import prepare_reuse_state  # noqa: F401
from ..ops import sparse_decode as triton_sparse_decode  # noqa: F401
from ..ops import sparse_decode_reuse as triton_sparse_decode_reuse  # noqa: F401
from ..ops import sparse_decode_unnorm as triton_sparse_decode_unnorm  # noqa: F401
