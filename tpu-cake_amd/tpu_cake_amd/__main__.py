"""``python -m tpu_cake_amd``: the workload contract commands (``render-workload``, ``experiment``,
``list-workloads``) of ``tpu_cake_amd.contracts``."""

import sys

from .contracts import main

sys.exit(main())
