"""CPU oracle for the CacheBlend KV data-movement and selection path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
reference results are compared against (or the timed CPU baseline). The product
package never imports it.
"""

from .cacheblend_oracle import *  # noqa: F401,F403
