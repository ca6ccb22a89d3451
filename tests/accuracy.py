"""The float64 anchor shared by the whole-model tests: a device path and the
oracle (ferrum_core's f32 arithmetic restated) are both compared with the
exact float64 forward of the same model, so a device error that stays inside
a per-score bound but is systematically larger than the reference's own
rounding still fails."""
import numpy as np


def accuracy_against_f64(got, ref, exact, what, mean_factor=1.5, max_factor=2.0):
    """Over every score given, the device's mean and largest error against
    the float64 result must be at most mean_factor and max_factor times the
    oracle's own.  Prints and returns (gpu mean, oracle mean, gpu max,
    oracle max)."""
    exact = np.asarray(exact, np.float64)
    eg = np.abs(np.asarray(got, np.float64) - exact)
    eo = np.abs(np.asarray(ref, np.float64) - exact)
    stats = (float(eg.mean()), float(eo.mean()), float(eg.max()), float(eo.max()))
    print(f"{what}: |err| vs float64 mean gpu {stats[0]:.3e} oracle {stats[1]:.3e}; "
          f"max gpu {stats[2]:.3e} oracle {stats[3]:.3e}")
    assert stats[0] <= mean_factor * stats[1], (
        f"{what}: mean error {stats[0]:.3e} above {mean_factor}x the oracle's {stats[1]:.3e}")
    assert stats[2] <= max_factor * stats[3], (
        f"{what}: max error {stats[2]:.3e} above {max_factor}x the oracle's {stats[3]:.3e}")
    return stats
