"""Process-wide defaults of the drop-in modules (set through
gruboros_amd.mingru.set_default_compute_dtype / install_alias)."""

# activation dtype of a minLM built with compute_dtype=None; None keeps the
# parameters' dtype (the reference's fp32)
COMPUTE_DTYPE = None
