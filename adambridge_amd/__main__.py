"""``python -m adambridge_amd {build,info}`` (reference adambridge/__main__.py)."""

import sys

from .native import main

if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))
