"""Loads the ``_C`` extension; fails loudly when it has not been built."""
try:
    from . import _C  # noqa: F401
except ImportError as e:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "spira_amd native extension is missing: run `python -m spira_amd.build` "
        f"(needs hipcc and PyTorch-ROCm) -- {e}") from e
