"""Seeded VAE weights and input of the reference's own VAE test
(debug/test_vae.c: build_vae :140-248, make_input :250-255, rng_f :83-90),
regenerated in numpy so the oracle can be checked against that test's golden
encode checksum (test_encode_golden :292-309: 29.091131 +- 0.2 for seed 1,
z_channels 32, eps 1e-4, quant convs, a 32x32 input from seed 7).

The generator is the Numerical Recipes 64-bit LCG g <- g * 6364136223846793005
+ 1442695040888963407 with value ((float)(g >> 32) / 4294967295.0f) * 2 - 1,
drawn in the order build_vae allocates the weights; norms are 1, biases 0,
convolution weights the draw times 0.05. Writes an f32 safetensors file in the
diffusers layout that the loaders read."""
import numpy as np

A, C = np.uint64(6364136223846793005), np.uint64(1442695040888963407)
CHUNK = 1 << 20
MULT = [1, 2, 4, 4]


class Lcg:
    def __init__(self, seed):
        self.g = np.uint64(seed if seed else 0x9E3779B97F4A7C15)
        with np.errstate(over="ignore"):
            self.ak = np.cumprod(np.full(CHUNK, A, np.uint64))                  # A^1 .. A^n
            self.sk = np.cumsum(np.concatenate([[np.uint64(1)], self.ak[:-1]]))  # 1 + A + .. + A^(k-1)

    def floats(self, n):
        out = np.empty(n, np.float32)
        done = 0
        with np.errstate(over="ignore"):
            while done < n:
                k = min(CHUNK, n - done)
                g = self.ak[:k] * self.g + self.sk[:k] * C
                x = (g >> np.uint64(32)).astype(np.uint32)
                out[done:done + k] = (x.astype(np.float32) / np.float32(4294967295.0)) * np.float32(2.0) - np.float32(1.0)
                self.g = g[-1]
                done += k
        return out


def build_vae(seed=1, z=32, with_quant=True):
    """(name, f32 array) of every tensor, in build_vae's draw order."""
    rng = Lcg(seed)
    t = []

    def rand(name, shape):
        t.append((name, (rng.floats(int(np.prod(shape))) * np.float32(0.05)).reshape(shape)))

    def fill(name, n, v):
        t.append((name, np.full(n, v, np.float32)))

    def res(p, cin, cout):
        fill(p + ".norm1.weight", cin, 1.0)
        fill(p + ".norm1.bias", cin, 0.0)
        rand(p + ".conv1.weight", (cout, cin, 3, 3))
        fill(p + ".conv1.bias", cout, 0.0)
        fill(p + ".norm2.weight", cout, 1.0)
        fill(p + ".norm2.bias", cout, 0.0)
        rand(p + ".conv2.weight", (cout, cout, 3, 3))
        fill(p + ".conv2.bias", cout, 0.0)
        if cin != cout:
            rand(p + ".conv_shortcut.weight", (cout, cin, 1, 1))
            fill(p + ".conv_shortcut.bias", cout, 0.0)

    def attn(p, ch):
        fill(p + ".group_norm.weight", ch, 1.0)
        fill(p + ".group_norm.bias", ch, 0.0)
        for n in ("to_q", "to_k", "to_v", "to_out.0"):
            rand(p + f".{n}.weight", (ch, ch))
            fill(p + f".{n}.bias", ch, 0.0)

    rand("encoder.conv_in.weight", (128, 3, 3, 3))
    fill("encoder.conv_in.bias", 128, 0.0)
    for level in range(4):
        ch, prev = 128 * MULT[level], 128 * MULT[level - 1] if level else 128
        for r in range(2):
            res(f"encoder.down_blocks.{level}.resnets.{r}", prev if r == 0 and level else ch, ch)
    for i in range(3):
        ch = 128 * MULT[i]
        rand(f"encoder.down_blocks.{i}.downsamplers.0.conv.weight", (ch, ch, 3, 3))
        fill(f"encoder.down_blocks.{i}.downsamplers.0.conv.bias", ch, 0.0)
    res("encoder.mid_block.resnets.0", 512, 512)
    attn("encoder.mid_block.attentions.0", 512)
    res("encoder.mid_block.resnets.1", 512, 512)
    fill("encoder.conv_norm_out.weight", 512, 1.0)
    fill("encoder.conv_norm_out.bias", 512, 0.0)
    rand("encoder.conv_out.weight", (2 * z, 512, 3, 3))
    fill("encoder.conv_out.bias", 2 * z, 0.0)
    if with_quant:
        rand("quant_conv.weight", (2 * z, 2 * z, 1, 1))
        fill("quant_conv.bias", 2 * z, 0.0)
    rand("decoder.conv_in.weight", (512, z, 3, 3))
    fill("decoder.conv_in.bias", 512, 0.0)
    res("decoder.mid_block.resnets.0", 512, 512)
    attn("decoder.mid_block.attentions.0", 512)
    res("decoder.mid_block.resnets.1", 512, 512)
    for i in range(4):
        level = 3 - i
        ch, prev = 128 * MULT[level], 512 if level == 3 else 128 * MULT[level + 1]
        for r in range(3):
            res(f"decoder.up_blocks.{i}.resnets.{r}", prev if r == 0 else ch, ch)
    for i in range(3):
        ch = 128 * MULT[3 - i]
        rand(f"decoder.up_blocks.{i}.upsamplers.0.conv.weight", (ch, ch, 3, 3))
        fill(f"decoder.up_blocks.{i}.upsamplers.0.conv.bias", ch, 0.0)
    fill("decoder.conv_norm_out.weight", 128, 1.0)
    fill("decoder.conv_norm_out.bias", 128, 0.0)
    rand("decoder.conv_out.weight", (3, 128, 3, 3))
    fill("decoder.conv_out.bias", 3, 0.0)
    if with_quant:
        rand("post_quant_conv.weight", (z, z, 1, 1))
        fill("post_quant_conv.bias", z, 0.0)
    return t


def make_input(seed, H, W):
    """[3][H][W] in [-1, 1]"""
    return Lcg(seed).floats(3 * H * W).reshape(3, H, W)


GOLDEN_ENCODE_CHECKSUM = 29.091131   # sum of latent[i] * (i % 13 + 1), 32x32 input
GOLDEN_TOL = 0.2


def checksum(lat):
    lat = np.asarray(lat, np.float64).ravel()
    return float(np.sum(lat * (np.arange(lat.size) % 13 + 1)))
