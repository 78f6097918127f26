import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


class heartbeat:
    """Context manager for long host-side computations inside a test (the oracle's step at the benchmark's shapes):
    every `period` seconds it prints a progress line to stderr and rewrites heartbeat.txt in the output folder under
    the repository root, so a runner watching for output sees the test is alive even when pytest captures stdout."""

    def __init__(self, what, period=30.0):
        self.what, self.period = what, period

    def __enter__(self):
        import threading
        import time
        self._stop = threading.Event()
        t0 = time.time()

        def beat():
            path = os.path.join(ROOT, "gpurun_out", "heartbeat.txt")
            while not self._stop.wait(self.period):
                line = f"[{self.what}] still running after {time.time() - t0:.0f} s"
                print(line, file=sys.stderr, flush=True)
                try:
                    os.makedirs(os.path.dirname(path), exist_ok=True)
                    with open(path, "w") as f:
                        f.write(line + "\n")
                except OSError:
                    pass

        self._t = threading.Thread(target=beat, daemon=True)
        self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._t.join()
        return False
