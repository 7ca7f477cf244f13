"""UMA-QMoE MoE-operator hot path, MI355X-native (gfx950).

Python host side of libuma_qmoe_hip.so:

* ``custom_op`` — the ``uma_qmoe`` torch.library operators and pack registry;
* ``native_backend`` — the install-then-select HIP backends over the C ABI
  (``_native``);
* ``formats`` — the canonical Q4 / Q8 / BF16 weight encodings;
* ``packfile`` — ExpertPack / TargetPack reading (through the library's C++
  reader) and writing;
* ``route_trace`` — the reference's RouteTrace documents as routing input;
* ``qwen_host`` — the fixed-Qwen model host around the MoE block;
* ``evidence`` — the reference's evidence documents and oracle metrics;
* ``synthetic`` — the seeded benchmark layers.
"""

__version__ = "0.1.0"
