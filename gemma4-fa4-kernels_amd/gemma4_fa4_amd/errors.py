"""Typed failures of the MI355X attention path.

The hierarchy mirrors the reference (src/gemma4_fa4/h100.py:37-42):
``UnsupportedH100Path(RuntimeError)`` and
``GlobalBackwardBudgetExceeded(UnsupportedH100Path)``; the reference names are
kept as aliases so callers catching them keep working.
"""


class UnsupportedMI355XPath(RuntimeError):
    """Raised when an input would leave the validated MI355X contract."""


class GlobalBackwardBudgetExceeded(UnsupportedMI355XPath):
    """Raised before launch when guarded HBM cannot admit global backward."""


UnsupportedH100Path = UnsupportedMI355XPath
