"""GPU encoders (brik_quantize_q8/q4/q3, brik_f16_to_f32) and the conversion path built on them, through
the C ABI, against the oracle: every output byte must equal the CPU encoder's (quantizeQ* + packQ*,
q8web.ts:28-62, q4web.ts:28-66, q3web.ts:34-76).

Covers the reference's chunked-conversion check (kernels.ts:2461-2472: 51 groups in chunks of 256
elements, last chunk partial, byte-equal to one pass), inputs with NaN / infinities / zero and
constant groups / exact ties / values outside the f16 range, F16 and .brik-quant sources, a device
weight handle fed to the matmul, and a .brik file written from GPU-encoded tensors and read back.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import container as C
from brimkern_amd import layout
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_EALIGN
from brimkern_amd.engine import Engine
from helpers import Gpu, PLANES, normwise_rel

pytestmark = pytest.mark.gpu

FMTS = ["q8", "q4", "q3"]


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


@pytest.fixture()
def engine(ctx):
    e = Engine(ctx=ctx)
    yield e
    e.close()


def oracle_bytes(fmt, x):
    with np.errstate(invalid="ignore"):          # signalling NaNs widened to f64 by the oracle
        return getattr(O, f"pack_{fmt}")(*getattr(O, f"quantize_{fmt}")(np.asarray(x, np.float32)))


def adversarial(seed, groups):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(32 * groups) * rng.choice([1e-3, 1, 40], 32 * groups)).astype(np.float32)
    n = x.size
    x[5] = np.nan
    x[32:64] = np.nan
    x[64:96] = 0
    x[64], x[80] = -0.0, -0.0                                 # the first minimum is -0: min bits 0x8000
    x[96:128] = -7.25
    x[97] = x[99] = 0.0
    x[98] = -0.0
    x[130], x[140] = np.inf, -np.inf
    x[160:192] = np.round(x[160:192] * 4) / 4                 # exact ties at several scales
    x[192:224] = (np.arange(32) - 15.5) * 0.0625
    x[224:256] = 1e-30
    x[256:288] = 3e38
    x[288:320] = -np.inf
    # ties across the halves of a group (the encoders scan each 16-element half on its own lane): a
    # +0 minimum before a -0 one, a -0 maximum before a +0 one, a first half of NaN, and equal extremes
    # in both halves
    x[352:384] = 0.0
    x[372] = -0.0                                             # min stays +0 (the first zero)
    x[384:400], x[400:416] = -0.0, 0.0                         # max stays -0, min -0
    x[416:432], x[432:448] = np.nan, rng.standard_normal(16).astype(np.float32)
    x[448:480] = 2.5
    x[452], x[470] = -3.0, -3.0
    x[n - 32:] = rng.standard_normal(32).astype(np.float32) * 1e4
    if n >= 1024:
        # signalling NaNs (the encoders take v_min / v_max of quieted values: an unquieted one would
        # become the group's extreme): among values, as a group's first element, with either sign,
        # and a group of nothing else but one value
        xb = x.view(np.uint32)
        xb[512], xb[517], xb[522] = 0x7F800001, 0xFFA00000, 0x7FBFFFFF
        xb[544:576] = 0x7F800001
        x[560] = 1.5
    return x


def gpu_quantize(gpu, fmt, x):
    n = x.size
    src = gpu.up(x)
    out = gpu.ctx.alloc(max(layout.byte_length(fmt, n), 1))
    gpu.bufs.append(out)
    offs = layout.plane_offsets(fmt, n)
    gpu.ctx.quantize(fmt, src, [out.offset(offs[p][0]) for p in PLANES[fmt]], n)
    return gpu.ctx.download(out, np.uint8, layout.byte_length(fmt, n))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("groups", [1, 51, 1000, 40000])
def test_quantize_bytes_equal_cpu_encoder(gpu, fmt, groups):
    x = adversarial(10 + groups, max(groups, 16))[: 32 * groups]
    assert np.array_equal(gpu_quantize(gpu, fmt, x), oracle_bytes(fmt, x))


def group_slice(fmt, blob, n, g0, g1):
    """The packed bytes of groups [g0, g1) cut out of the packed blob of an n-element tensor."""
    planes = layout.split_blob(fmt, blob, n)
    per_group = {"codes": 32, "nib": 16, "lo": 8, "hi": 4, "sc": 2, "mn": 2}       # bytes per group
    cut = {k: v.view(np.uint8)[g0 * per_group[k]:g1 * per_group[k]].view(v.dtype) for k, v in planes.items()}
    return layout.pack(fmt, cut)


@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_large_grid_stride(gpu, fmt):
    # more groups than one launch covers (2048 blocks x 128 groups): blocks loop over the rest; the
    # oracle checks the first groups and the last ones, taken by a later pass
    groups = 4096 * 256 + 777
    x = (np.random.default_rng(3).standard_normal(32 * groups) * 2).astype(np.float32)
    got = gpu_quantize(gpu, fmt, x)
    for g0, g1 in ((0, 2000), (groups - 3000, groups)):
        assert np.array_equal(group_slice(fmt, got, x.size, g0, g1), oracle_bytes(fmt, x[32 * g0:32 * g1])), (g0, g1)


def test_quantize_rejects_bad_args(gpu):
    src = gpu.up(np.zeros(64 + 4, np.float32))
    out = gpu.up(np.zeros(256, np.uint8))
    with pytest.raises(BrikError) as e:
        gpu.ctx.quantize("q4", src, [out.offset(0), out.offset(64), out.offset(96)], 48)
    assert e.value.code == BRIK_EINVAL
    with pytest.raises(BrikError) as e:
        gpu.ctx.quantize("q4", src.offset(4), [out.offset(0), out.offset(64), out.offset(96)], 32)
    assert e.value.code == BRIK_EALIGN
    with pytest.raises(BrikError) as e:
        gpu.ctx.quantize("q3", src, [out.offset(0), None, out.offset(64), out.offset(96)], 32)
    assert e.value.code == BRIK_EINVAL
    gpu.ctx.quantize("q8", src, [out.offset(0), out.offset(64)], 0)          # n = 0: no-op


def test_f16_to_f32_matches_reference_decode(gpu):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for n in (65536, 65533, 7, 1):
        b = gpu.up(bits[:n])
        o = gpu.ctx.alloc(4 * n)
        gpu.bufs.append(o)
        gpu.ctx.f16_to_f32(b, o, n)
        got = gpu.ctx.download(o, np.float32, n)
        # kernels.ts:3213-3222: IEEE half, exponent 31 -> +-65504
        want = bits[:n].view(np.float16).astype(np.float32)
        top = ((bits[:n] >> 10) & 31) == 31
        want[top] = np.where(bits[:n][top] >> 15, -65504.0, 65504.0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n


@pytest.mark.parametrize("dtype", FMTS)
def test_quantize_to_bytes_chunked_equals_single_pass(engine, dtype):
    # kernels.ts:2461-2472: 32 * 51 elements in chunks of 256 (7 chunks, the last partial)
    x = adversarial(51, 51)
    one = engine.quantize_to_bytes("F32", x, x.size, dtype)
    many = engine.quantize_to_bytes("F32", x, x.size, dtype, chunk=256)
    assert np.array_equal(one, many)
    assert np.array_equal(one, oracle_bytes(dtype, x))
    odd = engine.quantize_to_bytes("F32", x, x.size, dtype, chunk=100)     # rounded down to 96
    assert np.array_equal(one, odd)


@pytest.mark.parametrize("dtype", ["q8", "q4"])
def test_quantize_to_bytes_f16_source(engine, dtype):
    rng = np.random.default_rng(21)
    h = (rng.standard_normal(32 * 300) * 5).astype(np.float16).view(np.uint16).copy()
    h[7], h[40], h[41] = 0x7C00, 0xFC00, 0x7E00                 # inf, -inf, NaN: decoded as +-65504
    h[100] = 0x0001                                               # the smallest subnormal
    got = engine.quantize_to_bytes("F16", h, h.size, dtype, chunk=1024)
    f = h.view(np.float16).astype(np.float32)
    top = ((h >> 10) & 31) == 31
    f[top] = np.where(h[top] >> 15, -65504.0, 65504.0)
    assert np.array_equal(got, oracle_bytes(dtype, f))


@pytest.mark.parametrize("src_fmt,dtype", [("q4", "q8"), ("q8", "q4"), ("q3", "q4"), ("q4", "q3")])
def test_quantize_to_bytes_brik_quant_source(engine, src_fmt, dtype):
    x = (np.random.default_rng(31).standard_normal(32 * 700) * 2).astype(np.float32)
    blob = oracle_bytes(src_fmt, x)
    got = engine.quantize_to_bytes({"q8": "Q8W", "q4": "Q4W", "q3": "Q3W"}[src_fmt], blob, x.size, dtype, chunk=2048)
    deq = getattr(O, f"dequant_{src_fmt}")(*layout.split_blob(src_fmt, blob, x.size).values())
    assert np.array_equal(got, oracle_bytes(dtype, deq))


@pytest.mark.parametrize("fmt", FMTS)
def test_device_handle_feeds_the_matmul(engine, gpu, fmt):
    K, N, M = 512, 300, 3
    w = (np.random.default_rng(41).standard_normal(N * K) * 0.5).astype(np.float32)
    x = np.random.default_rng(42).standard_normal(M * K).astype(np.float32)
    wb = gpu.up(w)
    h = engine.quantize(fmt, wb, N * K)
    try:
        blob = engine.ctx.download(h["_buf"], np.uint8, layout.byte_length(fmt, N * K))
        assert np.array_equal(blob, oracle_bytes(fmt, w))
        yb = engine.mm(gpu.up(x), h, M, K, N)
        gpu.bufs.append(yb)
        y = engine.ctx.download(yb, np.float32, M * N)
        planes = layout.split_blob(fmt, blob, N * K)
        r = getattr(O, f"matmul_t_{fmt}")(x, *planes.values(), M, K, N).ravel()
        assert normwise_rel(y, r) <= 1e-3
    finally:
        engine.ctx.free(h["_buf"])


def test_brik_file_from_gpu_encoded_tensors(engine, gpu):
    d, ffn = 256, 512
    rng = np.random.default_rng(51)
    src = {"blk.0.attn_q.weight": ("q8", (d, d)), "blk.0.ffn_down.weight": ("q3", (d, ffn)),
           "blk.1.ffn_up.weight": ("q4", (ffn, d)), "token_embd.weight": ("q4", (64, d))}
    tensors, values = [], {}
    for name, (fmt, shape) in src.items():
        x = rng.standard_normal(int(np.prod(shape))).astype(np.float32)
        values[name] = x
        tensors.append({"name": name, "dtype": fmt, "shape": list(shape), "nElems": x.size,
                        "bytes": engine.quantize_to_bytes("F32", x, x.size, fmt).tobytes()})
    tensors.append({"name": "output_norm.weight", "dtype": "f32", "shape": [d], "data": np.ones(d, np.float32)})
    manifest, shards = C.assemble_brik({"name": "t"}, {"d": d}, {"template": "", "stopTokenIds": []},
                                       {"kind": "hf-hub", "id": "x"}, tensors)
    f = C.serialize_brik(manifest, shards)
    p = C.parse_brik(f)
    for name, (fmt, (N, K)) in src.items():
        e, b = C.tensor_bytes(p, name)
        assert bytes(b) == bytes(oracle_bytes(fmt, values[name]))
        h = engine.weight_from_container(p, name)
        try:
            x = rng.standard_normal(K).astype(np.float32)
            yb = engine.mm(gpu.up(x), h, 1, K, N)
            gpu.bufs.append(yb)
            y = engine.ctx.download(yb, np.float32, N)
            planes = layout.split_blob(fmt, np.frombuffer(b, np.uint8), N * K)
            r = getattr(O, f"matmul_t_{fmt}")(x, *planes.values(), 1, K, N).ravel()
            assert normwise_rel(y, r) <= 1e-5
        finally:
            engine.ctx.free(h["_buf"])
