"""The CPU oracle (both transcendental variants) against the reference's golden fixtures."""
import pytest

import golden_checks as gc

CHECKS = [gc.check_adam, gc.check_projection_fwd, gc.check_projection_bwd, gc.check_sh,
          gc.check_isect_sort_offsets, gc.check_raster_fwd, gc.check_raster_bwd, gc.check_ssim,
          gc.check_relocation, gc.check_perturb, gc.check_rng]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_matches_goldens(any_oracle, check):
    check(any_oracle)
