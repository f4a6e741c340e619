"""Host-side layout helpers of the flash core (CPU): every element lands where the documented
index formula of ``ffk_flash_attention_bias`` puts it."""
import torch

from foldforge_amd import kernels


def test_blocked_bias_follows_the_register_order():
    B, H, n = 1, 2, 64
    bias = torch.arange(B * H * n * n, dtype=torch.float32).reshape(B, H, n, n)
    blk = kernels.blocked_bias(bias)
    nb = n // 32
    assert blk.shape == (B * H, nb, nb, 4, 64, 4)
    flat = blk.reshape(-1)
    g = torch.Generator().manual_seed(3)
    for _ in range(200):
        bh = int(torch.randint(B * H, (1,), generator=g))
        j = int(torch.randint(n, (1,), generator=g))
        k = int(torch.randint(n, (1,), generator=g))
        kk = k % 32
        v, gg, e = kk // 8, (kk // 4) % 2, kk % 4
        lane = 32 * gg + j % 32
        index = ((((bh * nb + j // 32) * nb + k // 32) * 4 + v) * 64 + lane) * 4 + e
        assert flat[index] == bias.reshape(B * H, n, n)[bh, j, k]


def test_flash_v_layout_blocks_keys_and_swaps_key_bits_2_and_3():
    vt = torch.arange(2 * 32 * 64, dtype=torch.float32).reshape(2, 32, 64)
    out = kernels.flash_v_layout(vt)
    assert out.shape == (2, 2, 32, 32)
    flat = out.reshape(2, -1)
    for s in range(64):
        key = (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1)
        for d in (0, 7, 31):
            # the documented index: block s / 32, row d, slot s % 32
            assert flat[1, (s // 32) * 32 * 32 + d * 32 + s % 32] == vt[1, d, key]
    # within each 16-group: stored slots 0-3, 4-7, 8-11, 12-15 hold keys 0-3, 8-11, 4-7, 12-15
    assert out[0, 0, 0, :16].tolist() == [float(x) for x in [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]]
    # the second block holds keys 32 .. 63 of the same rows
    assert out[0, 1, 0, :4].tolist() == [32.0, 33.0, 34.0, 35.0]
