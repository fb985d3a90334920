"""Progress lines of the long GPU tests.  pytest captures the test process's stdout and stderr at the file-descriptor
level, so a line printed by a test shows only when it fails; a long test (a full-depth decode checked against the CPU
oracle) would look silent to whatever supervises the run.  say() also appends each line, flushed, to
test_progress.log in the run-output folder at the repository root (ETXMK_PROGRESS_DIR overrides the folder)."""
import os
import sys
import time
from pathlib import Path

_LOG = Path(os.environ.get("ETXMK_PROGRESS_DIR") or Path(__file__).resolve().parents[1] / "gpurun_out") / "test_progress.log"


def say(*a):
    msg = " ".join(str(x) for x in a)
    print(msg, flush=True)
    sys.stdout.flush()
    try:
        _LOG.parent.mkdir(exist_ok=True)
        with open(_LOG, "a") as f:
            f.write(f"{time.strftime('%H:%M:%S')} {msg}\n")
            f.flush()
    except OSError:
        pass
