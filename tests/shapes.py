"""Model shapes used by the tests."""
import qtts

# Small stacks with the real head_dim (128) and GQA ratio (2), sized so the
# oracle finishes in milliseconds.
TINY_TALKER = qtts.StackConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=320,
                               max_position=4096)
TINY_PREDICTOR = qtts.StackConfig(layers=2, hidden=128, heads=2, kv_heads=1, head_dim=128, inter=256, vocab=256,
                                  max_position=65536)
FULL_TALKER = qtts.TALKER_1P7B
FULL_PREDICTOR = qtts.PREDICTOR_1P7B

# Config-1 GEMV shapes (K -> N): gate/up, down, fused QKV.
GEMV_SHAPES = [(2048, 6144), (6144, 2048), (2048, 4096)]


def rel_err(got, ref):
    import numpy as np

    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(1e-30, float(np.max(np.abs(ref)))))
