import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Strict max-abs errors of the session's parity checks against the
    oracle, per dtype, with the tests that came closest to their tolerance."""
    from tests.helpers import PARITY_LOG

    if not PARITY_LOG:
        return
    tr = terminalreporter
    tr.write_line(f"parity summary: {len(PARITY_LOG)} checks of kernel outputs against the oracle "
                  "(strict max-abs error over every element)")
    for dtype in sorted({r[1] for r in PARITY_LOG}):
        rows = [r for r in PARITY_LOG if r[1] == dtype]
        worst = max(rows, key=lambda r: r[2])
        allowed = sum(r[4] for r in rows)
        line = (f"  {dtype}: {len(rows)} checks, largest error {worst[2]:.3e} (tolerance {worst[3]:.0e}) "
                f"in {worst[0]}")
        if allowed:
            line += (f"; {allowed} elements of output magnitude where half an ulp exceeds half the "
                     f"tolerance took that allowance, largest error among them "
                     f"{max(r[5] for r in rows):.3e}")
        tr.write_line(line)
    ranked = sorted(PARITY_LOG, key=lambda r: r[2] / r[3] if r[3] > 0 else 0.0, reverse=True)[:5]
    tr.write_line("  closest to tolerance: " + "; ".join(f"{r[0]} {r[2]:.2e}/{r[3]:.0e}" for r in ranked))
