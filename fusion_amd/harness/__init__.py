"""The whole-layer configuration harness and its measurement protocol and result schema
(`glm52/bench/bench_layer.py`, `glm52/bench/bench_layer_ab.py`, `glm52/common.py`)."""
