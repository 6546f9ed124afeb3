"""Reference name of the page scorer (cvsa/kernels/page_scores.py:77)."""
from ..ops import score_pages as triton_score_pages  # noqa: F401
