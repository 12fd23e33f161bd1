"""The benchmark's algorithmic byte counts and seeded layer ranks, on the CPU.

Per-layer bytes of the latent decode at the Llama-3.1-8B shape (B16, 8192
beacons, 4 sinks + 128 tail + the current token, 32/8 heads, d 128) follow
the closed form of the measurement contract: latent K/V rows, raw K/V rows,
q in, out, and U_K / W_V once -- 76,152,832 / 143,327,232 / 210,501,632 B at
ranks 16 / 32 / 48.  The Qwen2.5-14B shape adds eight query heads' q and out
rows and the two up-projection biases."""
import bench


def test_layer_bytes_match_the_closed_form():
    assert bench.layer_bytes(16, 16) == 76_152_832
    assert bench.layer_bytes(32, 32) == 143_327_232
    assert bench.layer_bytes(48, 48) == 210_501_632


def test_layer_bytes_count_each_tensor_once():
    B, NB, HKV, D, RAW = 16, 8192, 8, 128, 133
    for hq, bias in ((32, False), (40, True)):
        for r in (16, 32, 48):
            latent = B * NB * HKV * 2 * r * 2
            raw = B * RAW * HKV * D * 2 * 2
            q_out = B * 2 * hq * D * 2
            weights = HKV * D * 2 * r * 2 + (2 * HKV * D * 2 if bias else 0)
            assert bench.layer_bytes(r, r, hq, bias) == latent + raw + q_out + weights
    # the split kernel reads the rows and q; making its own operands it also reads U_K (and the K bias)
    assert bench.split_kernel_bytes(32, 32) == 143_327_232 - 16 * 32 * 128 * 2 - 8 * 128 * 64 * 2
    assert bench.fused_kernel_bytes(32, 32) == 143_130_624
    assert bench.fused_kernel_bytes(32, 32, 40, True) - bench.split_kernel_bytes(32, 32, 40) == 8 * 128 * 32 * 2 + 8 * 128 * 2


def test_layer_ranks_are_the_seeded_draw():
    """The sweep's ranks are drawn by seed 0; the headline line's config
    lists them."""
    assert bench.draw_ranks(32, 0) == [32, 32, 16, 32, 48, 32, 32, 32, 32, 32, 48, 16, 48, 16, 32, 16, 16, 48, 32, 48,
                                       48, 48, 16, 32, 16, 48, 16, 48, 32, 32, 48, 16]
    assert bench.draw_ranks(48, 0)[:32] == bench.draw_ranks(32, 0)
    assert bench.SHAPES['latent']['hq'] == 32 and bench.SHAPES['qwen']['hq'] == 40
