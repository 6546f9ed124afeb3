"""Reference names of the coverage / complement / merge entry points
(cvsa/kernels/coverage.py:99, :218, :329)."""
from ..ops import check_coverage as triton_check_coverage  # noqa: F401
from ..ops import compute_complement as triton_compute_complement  # noqa: F401
from ..ops import lse_merge as triton_lse_merge  # noqa: F401
