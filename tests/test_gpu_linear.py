"""GPU parity of the dense EXL3 linear (torch.ops.exl3xpu_C.linear and its C-ABI) against oracle/linear.py.

Outputs: rel-L2 <= 2e-3 after the same final rounding to the output dtype on both sides; the large-M path is compared
with the oracle's "large" variant (the fp16 GEMM output rounded before the output Hadamard). The reconstructed
weights are bit-exact."""
import numpy as np
import pytest
import torch

from oracle import exl3, linear as olin, synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _group(ck):
    from exl3xpu.linear import FusedGroup
    tr = torch.from_numpy(ck["trellis"])
    b = ck["bounds"]
    shards = [(tr[:, b[g] // 16:b[g + 1] // 16].contiguous(), torch.from_numpy(ck["suh"][g]),
               torch.from_numpy(ck["svh"][b[g]:b[g + 1]])) for g in range(len(b) - 1)]
    return FusedGroup(shards, "cuda", cb=ck["cb"])


def _x(seed, M, k, dtype):
    xf = exl3.bf16_to_f32(synth.activations(seed, M, k))
    if dtype == torch.float16:
        xf = xf.astype(np.float16).astype(np.float32)
    return xf, torch.from_numpy(xf).to("cuda", dtype)


def _round(ref, dtype):
    return torch.from_numpy(ref.astype(np.float32)).to(dtype).float().numpy()


@pytest.mark.parametrize("K", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("M", [1, 2, 3, 8])
def test_linear_small_vs_oracle(K, M):
    print(f"case linear small K={K} M={M}", flush=True)
    ck = olin.checkpoint(100 + K, 512, [256, 128, 128], K)         # three shards of one fused q/k/v-style group
    g = _group(ck)
    for dtype in (torch.bfloat16, torch.float16):
        xf, x = _x(7 * M + K, M, 512, dtype)
        y = g(x)
        torch.cuda.synchronize()
        assert y.dtype == dtype and tuple(y.shape) == (M, 512)
        r = _rel(y.float().cpu().numpy(), _round(olin.linear(xf, ck, "small"), dtype))
        assert r < TOL, (dtype, r)


@pytest.mark.parametrize("k,widths,K,M", [(2048, [1024, 1024], 3, 1), (4096, [512], 3, 3), (640, [384, 256], 5, 2),
                                          (128, [256], 4, 8), (2048, [256, 256, 512, 512], 2, 4)])
def test_linear_small_k_slices(k, widths, K, M):
    """The fused path over 1 to 8 K-slices of 512 rows, with a last slice that is partly past the end of k (640, 128:
    those waves add nothing), several shards: the last workgroup of every 128-column block sums the slices in order."""
    print(f"case linear small k={k} widths={widths} K={K} M={M}", flush=True)
    ck = olin.checkpoint(400 + k + K, k, widths, K)
    g = _group(ck)
    xf, x = _x(k + M, M, k, torch.bfloat16)
    y = g(x)
    torch.cuda.synchronize()
    r = _rel(y.float().cpu().numpy(), _round(olin.linear(xf, ck, "small"), torch.bfloat16))
    assert r < TOL, r


def test_linear_out_of_range_shard_gives_zero_columns():
    """A shard index outside [0, S) in shard_of_nb is never dereferenced: that block's columns come out zero and the
    other blocks are unchanged."""
    from exl3xpu.linear import C
    ck = olin.checkpoint(77, 256, [256, 256], 3)
    g = _group(ck)
    xf, x = _x(78, 2, 256, torch.bfloat16)
    good = g(x)
    bad_map = g.shard_of_nb.clone()
    bad_map[1] = 7
    y = C().linear(x, g.trellis, g.suh, g.svh, bad_map, g.bounds, g.K, g.cb, 8, 4096)
    torch.cuda.synchronize()
    assert not y[:, 128:256].float().any()
    assert torch.equal(y[:, :128], good[:, :128]) and torch.equal(y[:, 256:], good[:, 256:])


@pytest.mark.parametrize("K,M,slice_n", [(3, 9, 4096), (3, 300, 128), (4, 64, 192), (2, 33, 0), (6, 17, 256)])
def test_linear_large_vs_oracle(K, M, slice_n):
    """Above 8 rows: the input Hadamards, reconstructed fp16 weight slices (slice_n columns, 0 = whole groups) times xh
    of each shard group in the library GEMM, then the output Hadamard."""
    print(f"case linear large K={K} M={M} slice={slice_n}", flush=True)
    ck = olin.checkpoint(200 + K, 384, [256, 384, 128], K)
    g = _group(ck)
    xf, x = _x(11 + M, M, 384, torch.bfloat16)
    y = g(x, slice_n=slice_n)
    torch.cuda.synchronize()
    r = _rel(y.float().cpu().numpy(), _round(olin.linear(xf, ck, "large"), torch.bfloat16))
    assert r < TOL, r


def test_linear_small_threshold_and_shapes():
    """small_m_max picks the path (both agree with the oracle), batch dimensions are kept, bias is added, M = 0 is an
    empty result."""
    ck = olin.checkpoint(31, 256, [256], 3)
    g = _group(ck)
    xf, x = _x(5, 6, 256, torch.float16)
    ref = olin.linear(xf, ck, "small")
    y_small = g(x.view(2, 3, 256), small_m_max=8)
    y_large = g(x.view(2, 3, 256), small_m_max=1)
    bias = torch.full((256,), 0.5, device="cuda", dtype=torch.float16)
    y_bias = g(x, bias=bias)
    torch.cuda.synchronize()
    assert tuple(y_small.shape) == (2, 3, 256)
    assert _rel(y_small.reshape(6, 256).float().cpu().numpy(), _round(ref, torch.float16)) < TOL
    assert _rel(y_large.reshape(6, 256).float().cpu().numpy(), _round(olin.linear(xf, ck, "large"), torch.float16)) < TOL
    assert torch.allclose(y_bias.float(), y_small.reshape(6, 256).float() + 0.5, atol=2e-3)
    assert tuple(g(x[:0]).shape) == (0, 256)


@pytest.mark.parametrize("K", [2, 3, 5])
def test_reconstruct_bitexact(K):
    """exl3_reconstruct of a column range == the oracle's decode of the same tiles, bit for bit."""
    from exl3xpu.linear import C
    print(f"case reconstruct K={K}", flush=True)
    ck = olin.checkpoint(300 + K, 256, [512], K)
    ref = olin.weight(ck["trellis"], K).view(np.uint16)
    tr = torch.from_numpy(ck["trellis"]).cuda()
    for n0, n1 in ((0, 512), (16, 48), (128, 400)):
        w = torch.empty((256, n1 - n0), dtype=torch.float16, device="cuda")
        C().exl3_reconstruct(tr, w, n0, K, 2)
        torch.cuda.synchronize()
        assert np.array_equal(w.cpu().numpy().view(np.uint16), ref[:, n0:n1]), (n0, n1)


def test_had_in_had_out_vs_oracle():
    """exl3_had_in_rm: xh within one fp16 ulp of the oracle (butterfly order aside, equal almost everywhere);
    exl3_had_out_h: svh * H(y) / sqrt 128 within fp32 rounding."""
    from exl3xpu.linear import C
    ck = olin.checkpoint(41, 256, [128, 128], 3)
    xf, x = _x(3, 5, 256, torch.bfloat16)
    ref = olin.had_in(xf, ck["suh"])
    xh = torch.empty((2, 5, 256), dtype=torch.float16, device="cuda")
    C().exl3_had_in_rm(x, torch.from_numpy(ck["suh"]).cuda(), xh)
    y = torch.from_numpy(np.random.default_rng(2).standard_normal((5, 256)).astype(np.float16)).cuda()
    out = torch.empty((5, 256), dtype=torch.float32, device="cuda")
    C().exl3_had_out_h(y, torch.from_numpy(ck["svh"]).cuda(), out)
    torch.cuda.synchronize()
    got = xh.cpu().numpy()
    assert np.mean(got == ref) > 0.99
    assert np.max(np.abs(got.astype(np.float32) - ref.astype(np.float32))) <= np.max(np.abs(ref)) * 2.0 ** -10
    want = exl3.had_blocks(y.cpu().numpy().astype(np.float32)) * exl3.RSQRT128 * ck["svh"].astype(np.float32)
    assert np.allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6)


def test_linear_small_capi_fp32_out():
    """exl3_linear_small through the C-ABI: fp32 output with a row stride, the caller's zeroed workspace used by two
    calls in a row (4 rows, then 2), its counters left zero after each."""
    from exl3xpu import capi
    L = capi.lib()
    ck = olin.checkpoint(51, 1024, [512, 256], 4)
    k, n, S = 1024, 768, 2
    tr = torch.from_numpy(ck["trellis"]).cuda()
    suh = torch.from_numpy(ck["suh"]).cuda()
    svh = torch.from_numpy(ck["svh"]).cuda()
    sonb = torch.from_numpy(ck["shard_of_nb"]).cuda()
    ws_bytes = L.exl3_linear_workspace(4, k, n)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    for M, seed in ((4, 8), (2, 9)):
        xf, x = _x(seed, M, k, torch.bfloat16)
        out = torch.zeros((M, n + 64), dtype=torch.float32, device="cuda")
        capi.check(L.exl3_linear_small(x.data_ptr(), 1, k, M, k, n, tr.data_ptr(), 4, 2, suh.data_ptr(), S,
                                       svh.data_ptr(), sonb.data_ptr(), out.data_ptr(), 2, n + 64, ws.data_ptr(),
                                       ws_bytes, capi.stream_handle()), "linear_small")
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert _rel(got[:, :n], olin.linear(xf, ck, "small")) < TOL, M
        assert not got[:, n:].any()                               # nothing written past n in the padded rows
        assert not ws[:n // 128 * 4].any()                        # every arrival counter back at zero


def test_linear_small_in_graph_replays():
    """The fused small path captured in a HIP graph (the shared per-stream workspace and its counters) and replayed
    several times with new inputs and eager calls in between: every replay equals the eager result bit for bit."""
    ck = olin.checkpoint(71, 512, [256, 256], 3)
    g = _group(ck)
    xs = [_x(80 + i, 1, 512, torch.bfloat16)[1] for i in range(4)]
    x_static = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        g(x_static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static = g(x_static)
    for x in xs:
        want = g(x)                                               # eager, on the current stream
        torch.cuda.synchronize()
        x_static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_static, want)


def test_linear_small_two_graphs_on_one_capture_stream():
    """Two graphs captured one after another on torch's default capture stream, with no call on that stream before the
    first capture, replayed second-first and then alternately with eager calls in between: every replay equals the
    eager result bit for bit. Each capture zeroes the arrival counters of a workspace of its own inside the graph, so
    a replay never depends on which graph (or eager call) ran before it."""
    print("case linear small two graphs on one capture stream", flush=True)
    ck = olin.checkpoint(72, 512, [256, 256], 3)
    g = _group(ck)
    xs = [_x(90 + i, 1, 512, torch.bfloat16)[1] for i in range(3)]
    xa, xb = xs[0].clone(), xs[1].clone()
    ga, gb = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(ga):
        ya = g(xa)
    with torch.cuda.graph(gb):
        yb = g(xb)
    torch.cuda.synchronize()
    want_a, want_b, want_c = g(xs[0]), g(xs[1]), g(xs[2])         # eager, on the current stream
    torch.cuda.synchronize()
    for rep in range(3):
        gb.replay()
        torch.cuda.synchronize()
        assert torch.equal(yb, want_b), rep
        ga.replay()
        torch.cuda.synchronize()
        assert torch.equal(ya, want_a), rep
        yc = g(xs[2])
        torch.cuda.synchronize()
        assert torch.equal(yc, want_c), rep


@pytest.mark.parametrize("K", [4, 6])
@pytest.mark.parametrize("cb", [0, 1])
def test_codebooks_3inst_mcg_vs_oracle(K, cb):
    """The 3inst (0) and mcg (1) codebooks at K = 4 and 6: reconstructed weights bit-exact, the fused path at 1, 3 and
    8 rows over one K-slice (k = 512) and over four (k = 2048, the tagged hand-off), and the large-M path, against the
    oracle."""
    from exl3xpu.linear import C
    print(f"case codebook cb={cb} K={K}", flush=True)
    ck = olin.checkpoint(500 + 10 * cb + K, 512, [256, 128, 128], K, cb)
    ref = olin.weight(ck["trellis"], K, cb).view(np.uint16)
    tr = torch.from_numpy(ck["trellis"]).cuda()
    w = torch.empty((512, 512), dtype=torch.float16, device="cuda")
    C().exl3_reconstruct(tr, w, 0, K, cb)
    torch.cuda.synchronize()
    assert np.array_equal(w.cpu().numpy().view(np.uint16), ref)
    g = _group(ck)
    for M in (1, 3, 8):
        xf, x = _x(M + K + cb, M, 512, torch.bfloat16)
        y = g(x)
        torch.cuda.synchronize()
        r = _rel(y.float().cpu().numpy(), _round(olin.linear(xf, ck, "small"), torch.bfloat16))
        assert r < TOL, (M, r)
    xf, x = _x(40 + K, 21, 512, torch.float16)
    y = g(x, slice_n=256)
    torch.cuda.synchronize()
    r = _rel(y.float().cpu().numpy(), _round(olin.linear(xf, ck, "large"), torch.float16))
    assert r < TOL, ("large", r)
    ck4 = olin.checkpoint(600 + 10 * cb + K, 2048, [512, 256], K, cb)
    g4 = _group(ck4)
    xf, x = _x(70 + K, 2, 2048, torch.bfloat16)
    y = g4(x)
    torch.cuda.synchronize()
    r = _rel(y.float().cpu().numpy(), _round(olin.linear(xf, ck4, "small"), torch.bfloat16))
    assert r < TOL, ("k-slices", r)


@pytest.mark.parametrize("cb", [0, 1])
def test_reconstruct_codebooks_nearly_all_states(cb):
    """3inst / mcg through the GPU decoder over 4,096 random K=4 tiles (1M values; with this seed every one of the
    65,536 states occurs): every value equals the oracle's, bit for bit."""
    from exl3xpu.linear import C
    K = 4
    rng = np.random.default_rng(90 + cb)
    tr = rng.integers(0, 1 << 16, size=(64, 64, 16 * K), dtype=np.uint16).view(np.int16)
    ref = olin.weight(tr, K, cb).view(np.uint16)
    w = torch.empty((1024, 1024), dtype=torch.float16, device="cuda")
    C().exl3_reconstruct(torch.from_numpy(tr).cuda(), w, 0, K, cb)
    torch.cuda.synchronize()
    assert np.array_equal(w.cpu().numpy().view(np.uint16), ref)
    assert len(np.unique(exl3.tile_states(exl3.trellis_words(tr), K))) == 65536


@pytest.mark.parametrize("K", [4, 6])
def test_linear_int8_route_vs_oracle(K):
    """exl3_set_int8(1): above 16 rows, mul1 at K = 4 / 6 takes the W8A8 route. Its integer parts (xq, the row scales
    sx, the int8 weights) equal the oracle's bit for bit through the C-ABI; its output matches the oracle's W8A8
    restatement (rel-L2 2e-3: only the float steps after the exact integer GEMM differ) and the fp16 route within the
    int8 quantization error. At 16 rows, at K = 3 and with the switch off the fp16 route runs, bit-identical."""
    from exl3xpu import capi
    from exl3xpu.linear import C
    print(f"case int8 route K={K}", flush=True)
    L = capi.lib()
    ck = olin.checkpoint(700 + K, 512, [256, 128, 128], K)
    g = _group(ck)
    M, S = 40, 3
    xf, x = _x(80 + K, M, 512, torch.bfloat16)
    xq = torch.empty((S, M, 512), dtype=torch.int8, device="cuda")
    sx = torch.empty((S, M), dtype=torch.float32, device="cuda")
    wq = torch.empty((512, 384), dtype=torch.int8, device="cuda")
    capi.check(L.exl3_had_in_q8(x.data_ptr(), 1, x.stride(0), M, 512, g.suh.data_ptr(), S, xq.data_ptr(),
                                sx.data_ptr(), M, capi.stream_handle()), "had_in_q8")
    capi.check(L.exl3_reconstruct_q8(g.trellis.data_ptr(), 512, 512, 128, 512, K, wq.data_ptr(),
                                     capi.stream_handle()), "reconstruct_q8")
    torch.cuda.synchronize()
    rq, rs = olin.q8_act(xf, ck["suh"])
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(wq.cpu().numpy(), olin.q8_weight(ck["trellis"], K)[:, 128:])
    y16, y16_16 = g(x), g(x[:16])
    C().exl3_set_int8(1)
    try:
        y8, y8_16 = g(x), g(x[:16])
        ck3 = olin.checkpoint(710, 512, [256], 3)
        g3 = _group(ck3)
        y3_on = g3(x)
        torch.cuda.synchronize()
    finally:
        C().exl3_set_int8(0)
    y3_off = g3(x)
    torch.cuda.synchronize()
    r = _rel(y8.float().cpu().numpy(), _round(olin.linear_q8(xf, ck), torch.bfloat16))
    assert r < TOL, r
    r16 = _rel(y8.float().cpu().numpy(), y16.float().cpu().numpy())
    assert 1e-3 < r16 < 3e-2, r16
    assert torch.equal(y8_16, y16_16) and torch.equal(y3_on, y3_off)


@pytest.mark.parametrize("k", [1024, 4096, 16512])
def test_had_in_q8_row_lengths_bitexact(k):
    """The int8 input Hadamard over rows of 8, 32 and 129 blocks (blocks held in registers, 1 and 4 per wave, and
    the recomputing kernel for rows longer than 16,384): xq and the row scales equal the oracle's bit for bit."""
    from exl3xpu import capi
    print(f"case had_in_q8 k={k}", flush=True)
    L = capi.lib()
    ck = olin.checkpoint(720, k, [128, 128], 4)
    g = _group(ck)
    M, S = 17, 2
    xf, x = _x(81, M, k, torch.float16)
    xq = torch.empty((S, M + 3, k), dtype=torch.int8, device="cuda")
    sx = torch.empty((S, M + 3), dtype=torch.float32, device="cuda")
    capi.check(L.exl3_had_in_q8(x.data_ptr(), 0, x.stride(0), M, k, g.suh.data_ptr(), S, xq.data_ptr(),
                                sx.data_ptr(), M + 3, capi.stream_handle()), "had_in_q8")
    torch.cuda.synchronize()
    rq, rs = olin.q8_act(xf, ck["suh"])
    assert np.array_equal(xq[:, :M].cpu().numpy(), rq)
    assert np.array_equal(sx[:, :M].cpu().numpy().view(np.uint32), rs.view(np.uint32))
