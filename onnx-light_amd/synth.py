"""Synthetic inputs for the five benchmark configurations.

Draws use the reference's deterministic generator (canonical SplitMix64 and
its samplers, core/runtime/kernels/random.cc:32-106), vectorised with numpy:
the i-th draw of a stream seeded with s is mix(s + (i+1)*0x9E3779B97F4A7C15).
Seeds are 1000*config + tensor index; config 1's A uses seed 0.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64_draws(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Draws start..start+n-1 of the SplitMix64 stream seeded with `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Rand: (x >> 11) * 2^-53 in double."""
    return (splitmix64_draws(seed, n, start) >> np.uint64(11)).astype(np.float64) * (1.0 / 2.0**53)


def rand_int(low: int, high: int, seed: int, n: int) -> np.ndarray:
    """RandInt: uniform integers in [low, high), rejecting draws at or above
    2^64 - (2^64 mod span)."""
    span = high - low
    limit = (2**64 - (2**64 % span)) % 2**64
    x = splitmix64_draws(seed, n)
    if limit and np.any(x >= np.uint64(limit)):
        # a rejection shifts every later draw: replay sequentially
        out = np.empty(n, np.int64)
        i, j = 0, 0
        while i < n:
            v = int(splitmix64_draws(seed, 1, j)[0])
            j += 1
            if v < limit:
                out[i] = v % span + low
                i += 1
        return out
    return (x % np.uint64(span)).astype(np.int64) + low


def randn(seed: int, n: int, chunk: int = 1 << 20) -> np.ndarray:
    """Randn: sum of 12 uniforms minus 6, accumulated in draw order."""
    out = np.empty(n, np.float64)
    for c0 in range(0, n, chunk):
        c = min(chunk, n - c0)
        u = uniform(seed, 12 * c, 12 * c0).reshape(c, 12)
        acc = np.zeros(c, np.float64)
        for j in range(12):
            acc = acc + u[:, j]
        out[c0:c0 + c] = acc - 6.0
    return out


# ---- the same draws with torch (any device; bit-identical to the numpy path) --

def _torch_u64(v: int):
    """A 64-bit pattern as a torch int64 value (two's complement)."""
    return v - (1 << 64) if v >= 1 << 63 else v


def _lsr(z, k: int):
    """Logical right shift of int64 patterns (torch shifts arithmetically)."""
    return (z >> k) & ((1 << (64 - k)) - 1)


def splitmix64_draws_torch(seed: int, n: int, start: int = 0, device="cpu"):
    """splitmix64_draws as torch int64 bit patterns.  int64 products wrap
    modulo 2^64 like the uint64 ones, and XOR / masked shifts act on the bit
    patterns, so the draws are the same 64-bit values."""
    import torch
    idx = torch.arange(start + 1, start + n + 1, dtype=torch.int64, device=device)
    z = _torch_u64(seed) + idx * _torch_u64(int(GAMMA))
    z = (z ^ _lsr(z, 30)) * _torch_u64(int(_M1))
    z = (z ^ _lsr(z, 27)) * _torch_u64(int(_M2))
    return z ^ _lsr(z, 31)


def randn_torch(seed: int, n: int, device="cpu", chunk: int = 1 << 22):
    """randn (float64) computed with torch on `device`: the same uniforms
    ((x >> 11) * 2^-53) summed in the same order."""
    import torch
    out = torch.empty(n, dtype=torch.float64, device=device)
    for c0 in range(0, n, chunk):
        c = min(chunk, n - c0)
        u = (_lsr(splitmix64_draws_torch(seed, 12 * c, 12 * c0, device), 11).to(torch.float64)
             * (1.0 / 2.0**53)).view(c, 12)
        acc = torch.zeros(c, dtype=torch.float64, device=device)
        for j in range(12):
            acc = acc + u[:, j]
        out[c0:c0 + c] = acc - 6.0
    return out


def config4_torch(device, scale: float = 1.0) -> dict:
    """Configuration 4's inputs as torch tensors on `device` (the bench draws
    them on the GPU: 700 M uniforms take half a minute in numpy): w uint8
    fp8e4m3fn codes [4096, 14336], scale float32 [14336], a bfloat16
    [M, 4096].  Equal to config_inputs(4) bit for bit."""
    import torch
    K, N, M = 4096, 14336, max(1, int(4096 * scale))
    w = randn_torch(4000, K * N, device).to(torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).view(K, N)
    s = torch.from_numpy((0.005 + 0.045 * uniform(4001, N)).astype(np.float32)).to(device)
    a = randn_torch(4002, M * K, device).to(torch.float32).to(torch.bfloat16).view(M, K)
    return {"w": w, "scale": s, "a": a}


def pack_int4(values: np.ndarray) -> np.ndarray:
    """Two 4-bit values per byte, low nibble = even flat index."""
    v = np.asarray(values, np.int64).reshape(-1) & 0xF
    if v.size % 2:
        v = np.concatenate([v, np.zeros(1, np.int64)])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


CONFIGS = {
    1: "MatMulInteger u8[64,256] x s8[256,128], a_zp=128, b_zp=0 -> i32[64,128] (CPU plumbing case)",
    2: "QLinearMatMul u8[2048,4096] x s8[4096,4096] -> u8[2048,4096]",
    3: "DequantizeLinear(int4 [4096,11008], block 32 on K, fp16 scales) -> MatMul fp16[8,4096]",
    4: "DequantizeLinear(fp8e4m3fn [4096,14336], fp32 per-column scale) -> Cast bf16 -> MatMul bf16[4096,4096]",
    5: "MatMulInteger s8[32,512,64] x s8[32,64,512], per-row/per-column int8 zero points -> i32[32,512,512]",
}


def config_inputs(cfg: int, scale: float = 1.0) -> dict:
    """numpy inputs of configuration `cfg`.  `scale` < 1 shrinks M (rows of
    the activations) for quick parity runs; weights keep their full shape."""
    import torch
    if cfg == 1:
        a = rand_int(0, 256, 0, 64 * 256).astype(np.uint8).reshape(64, 256)
        b = rand_int(-128, 128, 1, 256 * 128).astype(np.int8).reshape(256, 128)
        return {"a": a, "b": b, "a_zp": np.array(128, np.uint8), "b_zp": np.array(0, np.int8)}
    if cfg == 2:
        M = max(1, int(2048 * scale))
        a = rand_int(0, 256, 2000, 2048 * 4096).astype(np.uint8).reshape(2048, 4096)[:M]
        b = rand_int(-128, 128, 2001, 4096 * 4096).astype(np.int8).reshape(4096, 4096)
        b_scale = np.float32(0.001 + 0.009 * uniform(2002, 1)[0])
        return {"a": np.ascontiguousarray(a), "a_scale": np.array(0.02, np.float32),
                "a_zp": np.array(128, np.uint8), "b": b, "b_scale": np.array(b_scale, np.float32),
                "b_zp": np.array(0, np.int8), "y_scale": np.array(0.05, np.float32),
                "y_zp": np.array(128, np.uint8)}
    if cfg == 3:
        K, N, bs = 4096, 11008, 32
        x = randn(3000, 8 * K).astype(np.float32).astype(np.float16).reshape(8, K)
        w = rand_int(-8, 8, 3001, K * N).reshape(K, N)
        s = (0.002 + 0.018 * uniform(3002, (K // bs) * N)).astype(np.float32).astype(np.float16)
        return {"a": x, "w_q": w.astype(np.int8), "w": pack_int4(w), "w_shape": (K, N),
                "scale": s.reshape(K // bs, N), "axis": 0, "block": bs}
    if cfg == 4:
        K, N, M = 4096, 14336, max(1, int(4096 * scale))
        wf = torch.from_numpy(randn(4000, K * N).astype(np.float32))
        w = wf.to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(K, N)
        s = (0.005 + 0.045 * uniform(4001, N)).astype(np.float32)
        af = torch.from_numpy(randn(4002, M * K).astype(np.float32))
        a = af.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).reshape(M, K)
        return {"a_bits": a, "w": w, "scale": s, "axis": 1}
    if cfg == 5:
        a = rand_int(-128, 128, 5000, 32 * 512 * 64).astype(np.int8).reshape(32, 512, 64)
        b = rand_int(-128, 128, 5001, 32 * 64 * 512).astype(np.int8).reshape(32, 64, 512)
        za = rand_int(-4, 5, 5002, 512).astype(np.int8)
        zb = rand_int(-4, 5, 5003, 512).astype(np.int8)
        return {"a": a, "b": b, "a_zp": za, "b_zp": zb}
    raise ValueError(f"unknown config {cfg}")
