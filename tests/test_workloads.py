"""CPU checks of the synthetic workload streams (tmac_synth_normal / _uniform in
libtmac_attn.so, tmac_gguf.cpp_amd/workloads.py).

The package's generator must give, bit for bit, the values of the oracle's
stream (oracle/tmac_oracle.c tmac_fill_normal, itself pinned by published
splitmix64 / xoshiro256** vectors in test_oracle.py), so that the benchmark and
the parity tests draw identical inputs.  The config 1 and config 2 inputs must
hash to the values stored in the golden fixtures.
"""
import os
import sys

import numpy as np
import pytest

import oracle
import tmac_attn
import workloads

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import gen_golden as gg  # noqa: E402


@pytest.mark.parametrize("seed", [0, 1, 3, 2000, 2**32 + 7, workloads.stream_id(3, workloads.K, 255), 2**64 - 1])
@pytest.mark.parametrize("n", [1, 2, 7, 1000])
def test_synth_normal_equals_oracle_stream(seed, n):
    np.testing.assert_array_equal(tmac_attn.synth_normal(seed, n), oracle.normal(seed, n))


def test_synth_uniform_equals_xoshiro_outputs():
    """u_i = (x_i >> 11) * 2^-53 over the oracle's xoshiro256** outputs of the same seed."""
    seed = workloads.stream_id(4, workloads.LENGTHS)
    state = oracle.splitmix64(seed, 4)
    xs = oracle.xoshiro256ss(state, 16)
    want = np.array([(x >> 11) * 2.0 ** -53 for x in xs])
    np.testing.assert_array_equal(tmac_attn.synth_uniform(seed, 16), want)


def test_synth_normal_moments():
    x = tmac_attn.synth_normal(12345, 1 << 20).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1) < 5e-3
    assert np.all(np.isfinite(x))


def test_config1_and_config2_inputs_match_golden_fixtures():
    q, k, v = workloads.c1()
    with np.load(os.path.join(HERE, "golden", "config1.npz"), allow_pickle=False) as f:
        assert gg.sha(q, k, v) == str(f["input_sha256"])
    q, kn, vn = workloads.c2(layers=2, steps=4)
    with np.load(os.path.join(HERE, "golden", "config2_slice.npz"), allow_pickle=False) as f:
        assert gg.sha(q, kn, vn) == str(f["input_sha256"])


def test_per_sequence_streams():
    """Sequence s of a per-sequence tensor is stream_id(config, tensor, s), filled in parallel."""
    n_seq, rows = 5, 33
    x = workloads.per_sequence(3, workloads.V, n_seq, rows, workloads.KVD)
    for s in range(n_seq):
        want = oracle.normal(workloads.stream_id(3, workloads.V, s), (rows, workloads.KVD))
        np.testing.assert_array_equal(x[s * rows:(s + 1) * rows], want)


def test_config4_lengths_and_pool():
    q, k, v, offs, lens = workloads.c4(n_seq=6, max_len=100)
    want = 1 + np.floor(tmac_attn.synth_uniform(workloads.stream_id(4, workloads.LENGTHS), 6) * 100)
    np.testing.assert_array_equal(lens, want.astype(np.int32))
    assert lens.min() >= 1 and lens.max() <= 100
    np.testing.assert_array_equal(offs, np.concatenate([[0], np.cumsum(lens[:-1])]))
    for s in range(6):
        np.testing.assert_array_equal(k[offs[s]:offs[s] + lens[s]],
                                      oracle.normal(workloads.stream_id(4, workloads.K, s), (lens[s], workloads.KVD)))
        np.testing.assert_array_equal(q[s], oracle.normal(workloads.stream_id(4, workloads.Q, s), workloads.QD))
    # the default config-4 draw: 16 lengths in [1, 32768]
    full = workloads.c4_lengths()
    assert full.size == 16 and full.min() >= 1 and full.max() <= 32768
