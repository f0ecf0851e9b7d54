"""linatt_amd: MI355X-native (gfx950 HIP) KATA-SPD attention and chunked
(gated) delta rule, drop-in for the reference's op modules.

Op modules (``linatt_amd.parallel_kata_attn``, ...) load the compiled
library ``linatt_amd/_lib/liblinatt_hip.so`` when imported and raise
``ImportError`` if it is missing (build: ``python -m linatt_amd.build``).
"""

__version__ = "0.1.0"
