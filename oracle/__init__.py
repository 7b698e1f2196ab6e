"""CPU oracle for the gated-DeltaNet (GDN) layer -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this
package, and only to check results (or as the timed CPU baseline). The product path (``zonos3-mini_amd``)
never imports it and has no CPU fallback.
"""

from .gdn_oracle import *  # noqa: F401,F403
