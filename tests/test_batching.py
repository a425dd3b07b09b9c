"""Host logic for packed ragged batches (no GPU)."""
import numpy as np
import pytest

from sys1_amd import batching


@pytest.mark.parametrize("seed", [0, 1, 2, 99])
def test_draw_lengths_matches_oracle_stream(orc, seed):
    for lo, hi, budget, exact in [(16, 512, 8192, False), (64, 2048, 8192, True),
                                  (32, 1024, 128, True), (32, 1024, 4096, True)]:
        a = batching.draw_lengths(seed, lo, hi, budget, exact)
        b = orc.pack_ragged(seed, lo, hi, budget, exact)
        np.testing.assert_array_equal(a, b)
        if exact:
            assert a.sum() == budget


def test_splitmix64_known_answers():
    # SplitMix64 with state 0: the first outputs of the published generator
    # (state advanced by the golden gamma before mixing).
    out = batching.splitmix64(0, np.arange(3))
    assert [int(v) for v in out] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_cu_seqlens_and_round_trip():
    lengths = [3, 1, 4]
    np.testing.assert_array_equal(batching.cu_seqlens(lengths), [0, 3, 4, 8])
    padded = np.arange(3 * 4 * 2, dtype=np.float32).reshape(3, 4, 2)
    packed = batching.pack_rows(padded, lengths)
    assert packed.shape == (8, 2)
    back = batching.unpack_rows(packed, lengths, 4, fill=-1)
    for b, l in enumerate(lengths):
        np.testing.assert_array_equal(back[b, :l], padded[b, :l])
        assert (back[b, l:] == -1).all()
    with pytest.raises(ValueError):
        batching.cu_seqlens([1, -1])
    with pytest.raises(ValueError):
        batching.draw_lengths(0, 0, 10, 100)


def test_empty_budget():
    assert batching.draw_lengths(3, 16, 512, 0).size == 0
    assert batching.cu_seqlens([]).tolist() == [0]


def test_positions_restart_per_sequence():
    from sys1_amd.batching import positions
    np.testing.assert_array_equal(positions([3, 1, 0, 2]), [0, 1, 2, 0, 0, 1])
    assert positions([]).size == 0
    p = positions([5, 4])
    assert p.dtype == np.int32
