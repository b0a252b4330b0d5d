"""Progress lines that reach the terminal while a test runs.

pytest captures a test's output until the test ends; a long GPU test would
then print nothing for minutes.  live() lifts the capture for one line.
"""

from __future__ import annotations

import sys

_capman = None


def attach(config) -> None:
    global _capman
    _capman = config.pluginmanager.getplugin("capturemanager")


def live(msg: str) -> None:
    if _capman is not None:
        with _capman.global_and_fixture_disabled():
            sys.stdout.write(msg + "\n")
            sys.stdout.flush()
    else:
        print(msg, flush=True)
