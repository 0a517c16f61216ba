"""CPU checks of the backend's construction contract (no kernel runs)."""

import pytest

from hcp_vllm_plugin_amd import ring_backend as rb


@pytest.mark.parametrize("head_size", [100, 260, 0])
def test_impl_rejects_head_sizes_the_paged_cache_reads_cannot_serve(head_size):
    # the paged cache is read in place in 16-byte pieces: a multiple of 8 up to 256
    with pytest.raises(NotImplementedError, match="head_size"):
        rb.HcpRingAttentionImpl(8, head_size, 0.1, 2)


@pytest.mark.parametrize("head_size", [8, 72, 128, 256])
def test_impl_accepts_supported_head_sizes(head_size):
    impl = rb.HcpRingAttentionImpl(8, head_size, 0.1, 2)
    assert impl.head_size == head_size and impl.num_queries_per_kv == 4
