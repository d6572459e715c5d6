#!/usr/bin/env python3
"""Entry point at the reference's path (mlx/scripts/harness.py): runs the
gfx950 harness in metalbench_amd/harness.py with the same arguments."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from metalbench_amd.harness import main  # noqa: E402

if __name__ == "__main__":
    sys.exit(main())
