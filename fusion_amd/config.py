"""GLM-5.2 MoE FFN block constants used by the MI355X path.

Values restate `glm52/config.py:15-50` of the reference (themselves copied from the public
GLM-5.2 `config.json`); only the ones the MoE block reads are kept here.
"""

from __future__ import annotations

HIDDEN_SIZE = 6144  # glm52/config.py:15
MOE_INTERMEDIATE_SIZE = 2048  # glm52/config.py:17
N_ROUTED_EXPERTS = 256  # glm52/config.py:22
N_SHARED_EXPERTS = 1  # glm52/config.py:23
NUM_EXPERTS_PER_TOK = 8  # glm52/config.py:24
ROUTED_SCALING_FACTOR = 2.5  # glm52/config.py:25
NORM_TOPK_PROB = True  # glm52/config.py:26
N_GROUP = 1  # glm52/config.py:29
TOPK_GROUP = 1  # glm52/config.py:30
RMS_NORM_EPS = 1e-5  # glm52/config.py:46

W13_N = 2 * MOE_INTERMEDIATE_SIZE  # glm52/config.py:63, [gate | up] along 2I
W2_K = MOE_INTERMEDIATE_SIZE  # glm52/config.py:64

H = HIDDEN_SIZE
I = MOE_INTERMEDIATE_SIZE
E = N_ROUTED_EXPERTS
TOPK = NUM_EXPERTS_PER_TOK

# Token counts of the benchmark configurations (BASELINE configs 0..4).
CONFIG_T = {0: 32, 1: 1, 2: 256, 3: 2048, 4: 8192}


def seed_for(T: int) -> int:
    """Seed convention of the reference benches: 1234 + T
    (`glm52/bench/bench_f04f05_norm_router.py:292`)."""
    return 1234 + T
