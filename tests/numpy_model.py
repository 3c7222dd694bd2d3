"""An independent float64 numpy statement of the LFM3 decode step, used only
to pin the oracle's composition (layer order, residuals, sandwich norms,
GQA mapping, ring slots). Vectorised and in double precision, so it shares
no summation order with the oracle; agreement within FP32 rounding shows
both follow reference.cpp:72-168."""
import ctypes

import numpy as np

import lfm3amd as L

_libm = ctypes.CDLL("libm.so.6")
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def powf(base, exponents):
    """glibc powf: reference.cpp's std::pow(float, float)."""
    return np.array([_libm.powf(base, float(e)) for e in np.asarray(exponents, np.float32)],
                    np.float32)


def deq(entry):
    data, typ, cols, rows = entry
    if typ == L.TYPE_Q8_0:
        return L.q8_dequant(data, rows, cols)
    return np.asarray(data, np.float64).reshape(rows, cols)


def rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


class NumpySession:
    def __init__(self, dims, weights, context, f16=True):
        self.d, self.w = dims, weights
        self.f16 = f16
        self.pos = 0
        self.conv = {}
        self.k, self.v, self.cap = {}, {}, {}
        self.mats = {}
        for i in range(dims.n_layers):
            t = dims.layer_type(i)
            if t == L.LAYER_CONV:
                self.conv[i] = np.zeros((dims.hidden, dims.conv_width - 1))
            else:
                cap = min(context, dims.window) if t == L.LAYER_SLIDING else context
                self.cap[i] = cap
                self.k[i] = np.zeros((cap, dims.kv_heads, dims.head_dim))
                self.v[i] = np.zeros((cap, dims.kv_heads, dims.head_dim))

    def m(self, entry):
        key = id(entry[0])
        if key not in self.mats:
            self.mats[key] = deq(entry)
        return self.mats[key]

    def rope(self, x, sliding):
        d = self.d
        D = d.head_dim
        i = np.arange(D // 2)
        theta = d.theta_swa if sliding else d.theta
        freq = powf(theta, np.float32(-2.0) * i.astype(np.float32) / np.float32(D))
        ang = (np.float32(self.pos) * freq).astype(np.float64)
        if not sliding:
            ang = ang / np.asarray(self.w.globals[3][0], np.float64)
        a, b = x[:, :D // 2], x[:, D // 2:]
        return np.concatenate([a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)], 1)

    def step(self, token):
        d, w = self.d, self.w
        H, D = d.hidden, d.head_dim
        x = self.m(w.globals[0])[token].copy()
        for i in range(d.n_layers):
            t = w.layers[i]
            z = rms(x, np.asarray(t[0][0], np.float64), d.eps)
            if d.layer_type(i) == L.LAYER_CONV:
                p = self.m(t[8]) @ z
                bx = p[:H] * p[2 * H:]
                taps = np.asarray(t[7][0], np.float64).reshape(H, d.conv_width)
                win = np.concatenate([self.conv[i], bx[:, None]], 1)
                y = (taps * win).sum(1) * p[H:2 * H]
                self.conv[i] = win[:, 1:]
                out = self.m(t[9]) @ y
            else:
                sliding = d.layer_type(i) == L.LAYER_SLIDING
                q = (self.m(t[10]) @ z).reshape(d.heads, D)
                k = (self.m(t[11]) @ z).reshape(d.kv_heads, D)
                v = (self.m(t[12]) @ z).reshape(d.kv_heads, D)
                g = self.m(t[15]) @ z
                qn, kn = np.asarray(t[13][0], np.float64), np.asarray(t[14][0], np.float64)
                q = np.stack([rms(h, qn, d.eps) for h in q])
                k = np.stack([rms(h, kn, d.eps) for h in k])
                q, k = self.rope(q, sliding), self.rope(k, sliding)
                cap = self.cap[i]
                slot = self.pos % cap
                if self.f16:
                    k = k.astype(np.float16).astype(np.float64)
                    v = v.astype(np.float16).astype(np.float64)
                self.k[i][slot], self.v[i][slot] = k, v
                first = max(0, self.pos + 1 - d.window) if sliding else 0
                ts = np.arange(first, self.pos + 1) % cap
                group = d.heads // d.kv_heads
                a = np.zeros((d.heads, D))
                for h in range(d.heads):
                    kh = h // group
                    s = self.k[i][ts, kh] @ q[h] / np.sqrt(D)
                    p_ = np.exp(s - s.max())
                    p_ /= p_.sum()
                    a[h] = (p_ @ self.v[i][ts, kh]) / (1 + np.exp(-g[h]))
                out = self.m(t[16]) @ a.reshape(-1)
            out = rms(out, np.asarray(t[2][0], np.float64), d.eps)
            x = x + out
            z = rms(x, np.asarray(t[1][0], np.float64), d.eps)
            gate, up = self.m(t[4]) @ z, self.m(t[5]) @ z
            h_ = gate / (1 + np.exp(-gate)) * up
            out = rms(self.m(t[6]) @ h_, np.asarray(t[3][0], np.float64), d.eps)
            x = x + out
        x = rms(x, np.asarray(w.globals[2][0], np.float64), d.eps)
        self.pos += 1
        return self.m(w.globals[0]) @ x
