import json
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("GI_PARITY_STATS")
    if not path:
        return
    from tests.helpers import PARITY_RECORD
    if PARITY_RECORD:
        Path(path).parent.mkdir(parents=True, exist_ok=True)
        Path(path).write_text(json.dumps(PARITY_RECORD, indent=1, sort_keys=True) + "\n")
