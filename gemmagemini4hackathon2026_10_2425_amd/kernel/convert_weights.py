#!/usr/bin/env python3
"""The kernel folder's convert script: --repo <hf_repo> (local HF cache) or
--src DIR, and --out <weights path>."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from gemmagemini4hackathon2026_10_2425_amd.weights import main  # noqa: E402

raise SystemExit(main())
