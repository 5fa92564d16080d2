"""bench.py's contract pieces that need no GPU: the roofline's per-launch traffic and MFMA-busy figures come from
the committed rocprofv3 summary of the default workload, looked up by the kernel names the trace prints. A
renamed kernel (a new template argument, say) would silently drop them from the bench line, so every kernel
bench.py reports a roofline for must be found in both of the summary's tables."""
import bench


def test_profiled_kernels_are_in_the_committed_summary():
    labels = ['noise_pop_block_qkv[block]', 'noise_pop_block[block]', 'noise_pop_head_ce',
              'noise_attention_fwd[window 1024]', 'noise_attention_fwd[window 2048]']
    for label in labels:
        traffic, busy = bench.profiled_traffic(label), bench.profiled_mfma_busy(label)
        assert traffic is not None and traffic > 0, label
        assert busy is not None and 0.0 < busy < 1.0, label


def test_dominant_kernel_traffic_is_at_least_its_algorithmic_bytes():
    # the block kernel with the next q/k/v moves at least y (1 KiB) + the residual (2 KiB) in and the residual
    # (2 KiB) + q, k, v (3 KiB) out per member-token: 8 KiB x 1024 x 2048
    assert bench.profiled_traffic('noise_pop_block_qkv[block]') >= 8 * 1024 * 1024 * 2048
