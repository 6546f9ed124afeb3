"""The reference's kernel entry points (cvsa.kernels.*.triton_*) bound to the
HIP implementations in cvsa.ops, so callers of the reference's kernel API
import unchanged."""
