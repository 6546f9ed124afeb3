"""Coverage-Verified Sparse Attention (CVSA) decode path for AMD MI355X.

Sparse attention as draft, coverage as acceptance criterion, and recovery on
low-coverage heads -- with the reference's Python API (cvsa.backend,
cvsa.lse_merge, cvsa.complement, cvsa.runtime) over hand-written gfx950 HIP
kernels (cvsa.ops -> libcvsa_hip.so).
"""
