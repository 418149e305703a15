"""Independent pin of the oracle's VAE decoder (orc_vae_decode, restating
ts_vae::decode, src/vae_decoder.cpp:62-124) against the Oobleck decoder
written with torch's own Conv1d / ConvTranspose1d in fp64 from the model's
definition (docs/ARCHITECTURE.md section 7): WNConv1d(latent -> 16 C, k7,
p3); per block SnakeBeta -> ConvTranspose1d(in -> out, k 2 s, stride s,
padding ceil(s / 2)) -> residual units of dilation 1, 3, 9; SnakeBeta ->
Conv1d(C -> 2, k7, p3, no bias). The transposed convolutions get PyTorch's
[IC, OC, K] kernel here and the converter's conv1d kernel (flipped along K,
channels swapped, convert/convert_vae.py:19-26) in the oracle, which runs the
reference's zero-stuffed conv1d formulation -- so the test pins that
formulation and the conversion together.

The oracle sums fp32 products in double; torch runs fp64: tolerance 1e-5
rel-L2 (measured 1e-6 .. 4e-6). Planted mistakes -- an unflipped kernel, the
padding s instead of s / 2, exp(beta) in place of exp(-beta), dilation 1
everywhere -- each move the result far outside it."""
import numpy as np
import pytest

from conftest import rel_l2

torch = pytest.importorskip("torch")
F = torch.nn.functional

TOL = 1e-5
TINY = dict(latent_dim=4, channels=4, out_channels=2, c_mults=[1, 2, 2, 3, 3], strides=[2, 4, 4, 8, 8],
            max_latent=8)


def torch_decode(W, cfg, latent, flip=True, pad_full=False, beta_sign=-1.0, dilations=(1, 3, 9)):
    """fp64 Oobleck decoder; W holds the oracle's (converted) tensors, the
    transposed-convolution kernels are turned back into PyTorch's layout"""
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    x = t(latent)[None]                                              # (1, L, T)

    def snake(x, p):
        a, b = t(W[p + ".alpha"])[None, :, None], t(W[p + ".beta"])[None, :, None]
        return x + torch.exp(beta_sign * b) * torch.sin(torch.exp(a) * x) ** 2

    x = F.conv1d(x, t(W["decoder.layers.0.weight"]), t(W["decoder.layers.0.bias"]), padding=3)
    strides = list(cfg["strides"])[::-1]
    for n in range(5):
        bp = f"decoder.layers.{n + 1}"
        s = strides[n]
        x = snake(x, bp + ".layers.0")
        wc = t(W[bp + ".layers.1.weight"])                           # converter's conv1d kernel [OC, IC, K]
        wt = (wc.flip(-1) if flip else wc).permute(1, 0, 2)          # back to ConvTranspose1d [IC, OC, K]
        x = F.conv_transpose1d(x, wt, t(W[bp + ".layers.1.bias"]), stride=s, padding=s if pad_full else (s + 1) // 2)
        for r, d in enumerate(dilations):
            rp = f"{bp}.layers.{r + 2}"
            h = snake(x, rp + ".layers.0")
            h = F.conv1d(h, t(W[rp + ".layers.1.weight"]), t(W[rp + ".layers.1.bias"]), padding=3 * d, dilation=d)
            h = snake(h, rp + ".layers.2")
            h = F.conv1d(h, t(W[rp + ".layers.3.weight"]), t(W[rp + ".layers.3.bias"]))
            x = x + h
    x = snake(x, "decoder.layers.6")
    x = F.conv1d(x, t(W["decoder.layers.7.weight"]), None, padding=3)
    return x[0].numpy()


def weights(tensors, seed):
    """conv kernels N(0, 1 / (K IC)), biases N(0, 0.02), snake parameters
    N(0, 0.1). (With N(0, 0.5) the residual stream grows to ~60 and
    sin(exp(alpha) x) turns the fp32 rounding of its argument into ~5e-5 of
    the output: a property of fp32, which this pin is not about.)"""
    out = {}
    for i, (name, ne) in enumerate(tensors):
        rng = np.random.default_rng([seed, i])
        shape = tuple(int(x) for x in reversed(ne))
        while len(shape) > 1 and shape[0] == 1:
            shape = shape[1:]
        sd = 1 / np.sqrt(ne[0] * ne[1]) if name.endswith(".weight") else 0.02 if name.endswith(".bias") else 0.1
        out[name] = (rng.standard_normal(shape) * sd).astype(np.float32)
    return out


@pytest.fixture(scope="module")
def tiny(orc):
    ov = orc.OracleVae(orc.vae_config(**TINY))
    W = weights(ov.tensors(), 5)
    for k, v in W.items():
        ov.set_tensor(k, v)
    return ov, W


def test_vae_tensor_inventory(tiny):
    ov, _ = tiny
    names = dict(ov.tensors())
    C = TINY["channels"]
    # block 1: c_mults[4] C -> c_mults[3] C channels, stride 8 (kernel 16);
    # block 5: c_mults[0] C -> C, stride 2 (decoder blocks run the multipliers
    # backwards, with 1 prepended)
    assert names["decoder.layers.1.layers.1.weight"] == (16, 3 * C, 3 * C)
    assert names["decoder.layers.5.layers.1.weight"] == (4, C, C)
    assert names["decoder.layers.3.layers.4.layers.1.weight"] == (7, 2 * C, 2 * C)
    assert names["decoder.layers.7.weight"] == (7, C, 2)
    assert "decoder.layers.7.bias" not in names
    assert len(names) == 2 + 5 * (4 + 3 * 8) + 3


@pytest.mark.parametrize("T", [1, 3, 5])
def test_vae_decode_matches_torch(tiny, T):
    ov, W = tiny
    rng = np.random.default_rng(T)
    lat = rng.standard_normal((TINY["latent_dim"], T)).astype(np.float32)
    got = ov.decode(lat)
    assert got.shape == (2, T * 2048)
    ref = torch_decode(W, TINY, lat)
    e = rel_l2(got, ref)
    print(f"orc_vae_decode vs torch fp64 (T={T}): rel-L2 {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("mistake", [dict(flip=False), dict(pad_full=True), dict(beta_sign=1.0),
                                     dict(dilations=(1, 1, 1))])
def test_vae_restatement_detects_mistakes(tiny, mistake):
    ov, W = tiny
    lat = np.random.default_rng(9).standard_normal((TINY["latent_dim"], 3)).astype(np.float32)
    got = ov.decode(lat)
    try:
        wrong = torch_decode(W, TINY, lat, **mistake)
    except RuntimeError:                       # a shape mismatch is a detected mistake too
        return
    e = rel_l2(got, wrong) if wrong.shape == got.shape else np.inf
    print(f"planted {mistake}: rel-L2 {e:.2e}")
    assert e > 100 * TOL
