"""A from-scratch torch (CPU, float32) Big-LaMa generator that mirrors
lama-rs/src/model.rs:135-207 with the state-dict names of the weight
container -- an implementation independent of the C oracle, used to pin the
oracle's whole-network composition (test infrastructure).

Only valid for power-of-two bottleneck planes: torch's FFT follows the usual
sign convention, while the reference CPU engine's Bluestein path (other
lengths) uses the opposite one.
"""
import numpy as np
import torch
import torch.nn.functional as F


def _ops(W):
    t = lambda n: torch.from_numpy(np.array(W[n], np.float32))  # noqa: E731

    def bn(y, p):
        return F.batch_norm(y, t(p + ".running_mean"), t(p + ".running_var"), t(p + ".weight"), t(p + ".bias"),
                            False, 0.0, 1e-5)

    def fourier_unit(y, p, st=None):
        b, c, h, w = y.shape
        ff = torch.fft.rfftn(y, dim=(-2, -1), norm="ortho")
        ff = torch.stack((ff.real, ff.imag), dim=2).reshape(b, 2 * c, h, w // 2 + 1)  # [c0.re, c0.im, ...]
        if st is not None:
            st.append(ff)
        ff = F.relu(bn(F.conv2d(ff, t(p + ".conv_layer.weight")), p + ".bn"))
        if st is not None:
            st.append(ff)
        ff = ff.reshape(b, c, 2, h, w // 2 + 1)
        return torch.fft.irfftn(torch.complex(ff[:, :, 0], ff[:, :, 1]), s=(h, w), dim=(-2, -1), norm="ortho")

    def spectral(y, p, st=None):
        f = F.relu(bn(F.conv2d(y, t(p + ".conv1.0.weight")), p + ".conv1.1"))
        if st is not None:
            st.append(f)
        s = f + fourier_unit(f, p + ".fu", st)
        if st is not None:
            st.append(s)
        return F.conv2d(s, t(p + ".conv2.weight"))

    return t, bn, spectral


def spectral_block(W, k, x):
    """FFC k's SpectralTransform (model.{5 + k//2}.conv{1 + k%2}) over x
    [384][h][w] -> (out, [f, spectrum, FU conv after BN + ReLU, f + ifft])."""
    _, _, spectral = _ops(W)
    st = []
    with torch.no_grad():
        y = spectral(torch.from_numpy(np.ascontiguousarray(x, np.float32))[None],
                     f"model.{5 + k // 2}.conv{1 + k % 2}.ffc.convg2g", st)
    return y[0].numpy(), [a[0].numpy() for a in st]


def forward(W, x):
    """W: {name: np.ndarray}; x: [4][h][w] -> (out [3][h][w], {step: activation})."""
    t, bn, spectral = _ops(W)
    steps = {}

    def conv(y, w, pad, stride):
        if pad:
            y = F.pad(y, (pad, pad, pad, pad), mode="reflect")
        return F.conv2d(y, w, stride=stride)

    def ffc(xl, xg, pf, pb):
        ol = conv(xl, t(pf + ".convl2l.weight"), 1, 1) + conv(xg, t(pf + ".convg2l.weight"), 1, 1)
        og = conv(xl, t(pf + ".convl2g.weight"), 1, 1) + spectral(xg, pf + ".convg2g")
        return F.relu(bn(ol, pb + ".bn_l")), F.relu(bn(og, pb + ".bn_g"))

    with torch.no_grad():
        y = torch.from_numpy(np.ascontiguousarray(x, np.float32))[None]
        y = F.pad(y, (3, 3, 3, 3), mode="reflect")
        steps[0] = y[0].numpy().ravel()
        y = F.relu(bn(F.conv2d(y, t("model.1.ffc.convl2l.weight")), "model.1.bn_l"))
        steps[1] = y[0].numpy().ravel()
        for i in (2, 3):
            y = F.relu(bn(conv(y, t(f"model.{i}.ffc.convl2l.weight"), 1, 2), f"model.{i}.bn_l"))
            steps[i] = y[0].numpy().ravel()
        xl = F.relu(bn(conv(y, t("model.4.ffc.convl2l.weight"), 1, 2), "model.4.bn_l"))
        xg = F.relu(bn(conv(y, t("model.4.ffc.convl2g.weight"), 1, 2), "model.4.bn_g"))
        steps[4] = torch.cat([xl, xg], 1)[0].numpy().ravel()
        for i in range(5, 23):
            a, b = ffc(xl, xg, f"model.{i}.conv1.ffc", f"model.{i}.conv1")
            a, b = ffc(a, b, f"model.{i}.conv2.ffc", f"model.{i}.conv2")
            xl, xg = xl + a, xg + b
            steps[i] = torch.cat([xl, xg], 1)[0].numpy().ravel()
        y = torch.cat([xl, xg], 1)
        steps[23] = y[0].numpy().ravel()
        for k, i in enumerate((24, 27, 30)):
            y = F.conv_transpose2d(y, t(f"model.{i}.weight"), t(f"model.{i}.bias"), stride=2, padding=1,
                                   output_padding=1)
            y = F.relu(bn(y, f"model.{i + 1}"))
            steps[24 + k] = y[0].numpy().ravel()
        y = F.pad(y, (3, 3, 3, 3), mode="reflect")
        steps[27] = y[0].numpy().ravel()
        y = torch.sigmoid(F.conv2d(y, t("model.34.weight"), t("model.34.bias")))
        steps[28] = y[0].numpy().ravel()
    return y[0].numpy(), steps
