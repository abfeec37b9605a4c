"""Python -> native shim (reference: source/spira/nn/functional/).

Every function calls the ``_C`` extension built from ``spira_amd/csrc``; there
is no CPU fallback: CPU tensors raise ``NotImplementedError`` and a missing
extension raises ``ImportError`` at import time.
"""
from .convolution import *  # noqa: F401,F403
from .indexing import *  # noqa: F401,F403
from .memory import *  # noqa: F401,F403
