import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "mini-gpt-inference_amd"), str(ROOT), str(Path(__file__).resolve().parent)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")


@pytest.fixture
def progress(request):
    """A function that writes one progress line to the terminal at once, past
    pytest's output capture (suspended for the write), so a test that runs
    for minutes keeps its run visibly alive."""
    capman = request.config.pluginmanager.getplugin("capturemanager")

    def emit(line: str) -> None:
        if capman is None:
            print(line, flush=True)
            return
        with capman.global_and_fixture_disabled():
            print(line, flush=True)

    return emit
