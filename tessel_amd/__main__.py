"""`python -m tessel_amd ...`: the tessel command line (tessel_amd.cli)."""

import sys

from tessel_amd.cli import main

sys.exit(main())
