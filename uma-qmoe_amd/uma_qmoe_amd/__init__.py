"""UMA-QMoE MoE-operator hot path, MI355X-native (gfx950).

Python host side of libuma_qmoe_hip.so: the ``uma_qmoe`` torch.library
operators (custom_op), the install-then-select performance backends
(native_backend), the canonical Q4/Q8/BF16 codecs (q4, target_pack) and the
seeded benchmark layers (synthetic).
"""

__version__ = "0.1.0"
