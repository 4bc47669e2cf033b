"""Scalar stage arithmetic on bit patterns, in Python integers, for the plan
encoder's fill folding (docs/reloc-typed-semantics.md sections 3.1-3.6).
Product code: independent of the test oracle."""
import math
import struct


def _f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits & 0xffffffff))[0]


def _bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def _shr_rne(v, s):
    if s <= 0:
        return v
    q, r, half = v >> s, v & ((1 << s) - 1), 1 << (s - 1)
    return q + (1 if (r > half or (r == half and q & 1)) else 0)


def f32_to_f16(bits):
    sign = (bits >> 16) & 0x8000
    mag = bits & 0x7fffffff
    exp = mag >> 23
    if exp == 0xff:
        return sign | (0x7e00 | ((mag >> 13) & 0x3ff) if mag & 0x7fffff else 0x7c00)
    if exp >= 113:
        h = _shr_rne(((exp - 112) << 23) | (mag & 0x7fffff), 13)
        return sign | min(h, 0x7c00)
    if exp == 0:
        return sign
    return sign | _shr_rne((mag & 0x7fffff) | 0x800000, 126 - exp)


def f16_to_f32(h):
    sign = (h & 0x8000) << 16
    e, m = (h >> 10) & 0x1f, h & 0x3ff
    if e == 0x1f:
        return sign | 0x7f800000 | (m << 13)
    if e:
        return sign | ((e + 112) << 23) | (m << 13)
    if not m:
        return sign
    lead = m.bit_length() - 1
    return sign | ((lead + 103) << 23) | (((m << (10 - lead)) & 0x3ff) << 13)


def f32_to_bf16(bits):
    if (bits & 0x7fffffff) > 0x7f800000:
        return ((bits >> 16) | 0x40) & 0xffff
    return ((bits + 0x7fff + ((bits >> 16) & 1)) >> 16) & 0xffff


def bf16_to_f32(b):
    return (b & 0xffff) << 16


def cast_bits(bits, src, dst):
    if src == "float32" and dst == "float16":
        return f32_to_f16(bits)
    if src == "float16" and dst == "float32":
        return f16_to_f32(bits)
    if src == "float32" and dst == "bfloat16":
        return f32_to_bf16(bits)
    if src == "bfloat16" and dst == "float32":
        return bf16_to_f32(bits)
    raise ValueError("unsupported cast %s -> %s" % (src, dst))


def _round_f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def quantize_bits(bits, scale_bits):
    """symmetric_rne: inv = fl32(1/scale); t = fl32(x*inv); clamp (NaN -> -128); rne."""
    inv = _round_f32(1.0 / _f32(scale_bits))
    x = _f32(bits)
    t = _round_f32(x * inv) if not math.isnan(x) else float("nan")
    if math.isnan(t):
        q = -128
    else:
        t = min(max(t, -128.0), 127.0)
        q = int(round(t))  # Python round(): ties to even
    return q & 0xff


def dequantize_bits(bits, scale_bits, zp):
    q = bits & 0xff
    q = q - 256 if q >= 128 else q
    return _bits(_round_f32(float(q - zp) * _f32(scale_bits)))
