"""Marker for GPU tests of code paths that have not run on a GPU yet: they
are skipped unless DS4HIP_RUN_UNVERIFIED=1, so a run that means to try them
asks for them explicitly and every other run leaves them out."""
import os

import pytest

ENABLED = os.environ.get("DS4HIP_RUN_UNVERIFIED") == "1"


def unverified(reason: str):
    return pytest.mark.skipif(not ENABLED, reason=f"{reason} (set DS4HIP_RUN_UNVERIFIED=1 to run it)")
