#!/usr/bin/env python3
"""The kernel folder's build script: compiles libmxdecode.so for gfx950 in the
package directory (hipcc)."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from gemmagemini4hackathon2026_10_2425_amd.build import main  # noqa: E402

raise SystemExit(main([]))
