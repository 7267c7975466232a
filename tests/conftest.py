import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Repeat every PARITY line the tests printed (pytest captures them under -q), one per line at the end of
    the run, so that the measured rel-L2, ulp and over-bar figures of each configuration reach the run's
    output tail."""
    lines = []
    for key in ("passed", "failed"):
        for rep in terminalreporter.stats.get(key, []):
            if getattr(rep, "when", "") != "call":
                continue
            for line in (rep.capstdout or "").splitlines():
                if line.startswith("PARITY"):
                    lines.append(f"{line}  [{rep.nodeid.split('::', 1)[-1]}]")
    if lines:
        terminalreporter.section(f"PARITY lines ({len(lines)})")
        for line in lines:
            terminalreporter.write_line(line)
