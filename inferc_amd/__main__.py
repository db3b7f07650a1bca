"""`python -m inferc_amd <command>`: the inferc commands (see inferc_amd.cli)."""
import sys

from .cli import main

sys.exit(main())
