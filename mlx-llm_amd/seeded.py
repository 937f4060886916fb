"""Seeded synthetic inputs: SplitMix64 (src/primitives/sampler.rs:40-60)
feeding Box-Muller in f64, cast to f32 -- the input generator the benchmark
configurations are specified with.  Draw i of a stream seeded s is
SplitMix64's output for the state s + i * 0x9E3779B97F4A7C15 (i from 1), so
a whole tensor is generated at once on the device with int64 arithmetic
(two's-complement wrap-around is the mod-2^64 arithmetic SplitMix64 uses).
Pairs of draws (u1 from the first, 53 bits, in (0, 1]; u2 from the second,
in [0, 1)) give z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1),
stored in that order; value = f32(mean + std * z)."""

_GOLDEN = 0x9E3779B97F4A7C15
_M1 = 0xBF58476D1CE4E5B9
_M2 = 0x94D049BB133111EB


def _i64(v: int) -> int:
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= 1 << 63 else v


def _lsr(torch, z, s: int):
    """Logical right shift of int64 bit patterns."""
    return (z >> s) & ((1 << (64 - s)) - 1)


def splitmix_u53(seed: int, n: int, device="cpu"):
    """The first n draws of the stream, each >> 11 (53-bit integers, int64)."""
    import torch

    i = torch.arange(1, n + 1, device=device, dtype=torch.int64)
    z = i * _i64(_GOLDEN) + _i64(seed)
    z = (z ^ _lsr(torch, z, 30)) * _i64(_M1)
    z = (z ^ _lsr(torch, z, 27)) * _i64(_M2)
    z = z ^ _lsr(torch, z, 31)
    return _lsr(torch, z, 11)


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0, device="cpu", chunk: int = 1 << 24):
    """n f32 values of N(mean, std) from the SplitMix64 stream `seed`."""
    import struct

    import torch

    # mean and std are f32 parameters widened to f64, as the reference's
    mean, std = (struct.unpack("f", struct.pack("f", v))[0] for v in (mean, std))
    out = torch.empty(n, dtype=torch.float32, device=device)
    pairs = (n + 1) // 2
    two_pi = 6.283185307179586476925286766559
    scale = 1.0 / 9007199254740992.0  # 2^-53
    for p0 in range(0, pairs, chunk):
        p1 = min(pairs, p0 + chunk)
        # draws 2 p0 .. 2 p1 - 1 of the stream: offset the counter by 2 p0
        u = splitmix_u53(_i64(seed + 2 * p0 * _GOLDEN), 2 * (p1 - p0), device).to(torch.float64)
        u1 = (u[0::2] + 1.0) * scale
        u2 = u[1::2] * scale
        r = torch.sqrt(-2.0 * torch.log(u1))
        z = torch.stack((r * torch.cos(two_pi * u2), r * torch.sin(two_pi * u2)), dim=1).reshape(-1)
        e0, e1 = 2 * p0, min(n, 2 * p1)
        out[e0:e1] = (mean + std * z[: e1 - e0]).to(torch.float32)
    return out


def choice(seed: int, k: int, count: int) -> list[int]:
    """count distinct indices in [0, k), in draw order: draw d of the stream
    seeded `seed` names index (d >> 11) mod k; repeats are skipped."""
    out, seen, n = [], set(), 0
    while len(out) < count:
        n += 4 * count
        for v in splitmix_u53(seed, n).tolist()[n - 4 * count:]:
            c = v % k
            if c not in seen:
                seen.add(c)
                out.append(c)
                if len(out) == count:
                    break
    return out
