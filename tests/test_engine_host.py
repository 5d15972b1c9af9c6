"""Host-side choices of the engine and harness that need no GPU."""
from stride_amd import harness


def test_one_kernel_attention_budget():
    """The one-kernel attention's LDS budget as the library computes it: 7360
    positions (115 pages) fit at head_dim 64 with 16-token KV pages, 7361 and 8192
    do not; 2816 positions (44 pages) fit at head_dim 128, 2817 do not. An engine
    asked for item_count = -1 beyond the budget keeps the item list."""
    pages = lambda ctx: (ctx + 63) // 64
    assert harness.attention_one_kernel_fits(pages(7360), 64, 16)
    assert not harness.attention_one_kernel_fits(pages(7361), 64, 16)
    assert not harness.attention_one_kernel_fits(pages(8192), 64, 16)
    assert harness.attention_one_kernel_fits(pages(2816), 128, 16)
    assert not harness.attention_one_kernel_fits(pages(2817), 128, 16)
    assert harness.attention_one_kernel_fits(pages(512), 64, 16)
