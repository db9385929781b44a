"""Settings of the randomised (hypothesis) GPU property tests.

By default each test draws its committed number of examples from a fixed
seed, so every run checks the same cases.  Two environment variables widen
the search without editing the tests:
  LA_PROPERTY_SCALE  multiplies every test's number of examples (e.g. 20);
  LA_PROPERTY_SEED   draws the examples from this seed instead of the fixed one.
"""
from __future__ import annotations

import os

from hypothesis import HealthCheck, seed, settings


def property_test(max_examples: int):
    """Decorator for a @given test: the settings above, then the seed."""
    scale = float(os.environ.get("LA_PROPERTY_SCALE", "1"))
    chosen = os.environ.get("LA_PROPERTY_SEED")
    # no example database either way: a run checks exactly the drawn cases
    conf = settings(max_examples=max(1, int(max_examples * scale)), deadline=None, derandomize=chosen is None,
                    database=None, suppress_health_check=list(HealthCheck))

    def wrap(test):
        test = conf(test)
        return seed(int(chosen))(test) if chosen is not None else test
    return wrap
