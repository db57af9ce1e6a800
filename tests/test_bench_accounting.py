"""The byte and FLOP accounting bench.py reports (CPU only): the algorithmic
bytes and FLOPs of the layer configurations (one expert 1,671,168 B, one
(token, expert) pair 6,291,456 FLOPs), kept apart from this build's own
intermediates."""
import bench


def test_expert_bytes():
    assert bench.MAT_BYTES == 557_056
    assert bench.EXPERT_BYTES == 1_671_168


def test_decode1_bytes():
    # 8 experts x (gate + up) + e4m3 x with its E8M0 scales
    alg, ovh = bench.kernel_bytes("gateup", 1, 8, False)
    assert alg == 8 * 2 * 557_056 + 2048 + 64
    assert ovh == 8 * 512 + 8 * 16          # h codes + scales written for the down
    alg, ovh = bench.kernel_bytes("down", 1, 8, False)
    assert alg == 8 * 557_056 + 8 * 512 + 8 * 16
    assert ovh == 8 * (2048 * 2 + 2048 // 16)
    layer, flops = bench.algorithmic(1, 8, False)
    assert layer == 8 * 1_671_168 + 2048 * 4 + 256 * 4 + 2048 * 2   # 13.38 MB
    assert flops == 8 * 6_291_456


def test_prefill_down_is_weights_plus_h():
    # 142.6 MB of weights + 17.3 MB of h; the staging is overhead
    alg, ovh = bench.kernel_bytes("down", 4096, 256, False)
    assert alg == 256 * 557_056 + 4096 * 8 * (512 + 16)
    assert abs(alg - 159.9e6) < 0.1e6
    assert ovh == 4096 * 8 * (2048 * 2 + 128)   # f16 staging + exponents
    assert bench.kernel_flops("gateup", 4096, False) == 4096 * 8 * 2 * 2048 * 1024
    assert bench.kernel_flops("down", 4096, False) == 4096 * 8 * 2 * 512 * 2048
