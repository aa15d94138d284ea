"""GPU: prana-graph over device buffers (prana_graph_*, prana-graph
lib.rs:25-220) against the oracle's kernels composed in the same order, every
node's value bit for bit:
  - the reference's graph tests (lib.rs:227-304): a tiny block, a quantized
    matmul node, an attention block, an unset input;
  - the CLI's demo block (prana-cli main.rs:276-315: GQA 4/2, norm, QKV, RoPE,
    causal attention, MLP, residuals);
  - larger rows (Q8 matmuls on the skinny and matrix-core paths, attention
    over 300 rows), shape mismatches, the cached-value semantics of execute,
    reset, inputs from device memory and set_input on a computed node."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def sinw(n, seed, scale=1.0):
    return (np.sin(np.arange(n, dtype=np.float32) * np.float32(seed)) * np.float32(scale)).astype(np.float32)


def test_tiny_block():
    # runs_a_tiny_block (lib.rs:227-249): x -> rmsnorm -> matmul -> add -> softmax
    dim = 32
    g = P.Graph()
    x = g.input(1)
    norm_w = np.ones(dim, np.float32)
    n = g.rmsnorm(x, norm_w, dim, 1e-5)
    w = sinw(dim * dim, 0.001)
    proj = g.matmul_f32(n, w, dim, dim)
    res = g.add(proj, x)
    out = g.softmax(res)
    xv = np.full(dim, 0.5, np.float32)
    g.set_input(x, xv, (1, dim))
    g.execute()
    probs = g.output_f32(out)
    assert probs.size == dim and abs(float(probs.sum()) - 1.0) < 1e-5
    # the oracle, op by op
    on = O.rmsnorm(xv[None, :], norm_w, 1e-5)
    op = O.Mat.f32(w.reshape(dim, dim)).apply(on)
    orr = (op + xv[None, :]).astype(np.float32)
    assert same_bits(g.output_f32(n), on) and same_bits(g.output_f32(proj), op)
    assert same_bits(g.output_f32(res), orr) and same_bits(probs, O.softmax(orr.ravel()))
    assert g.shape(n) == (1, dim) and g.shape(out) == (dim,) and g.shape(res) == (1, dim)


@pytest.mark.parametrize("n_tok", [1, 5, 12, 64, 100])
def test_quantized_matmul_node(n_tok):
    # quantized_matmul_node_works (lib.rs:251-262), then batches across the
    # decode, skinny and matrix-core paths
    dim, rows = 64, 96
    w = np.cos(np.arange(rows * dim, dtype=np.float32) * np.float32(0.002)).astype(np.float32).reshape(rows, dim)
    q, s = O.quantize_q8(w)
    g = P.Graph()
    x = g.input(n_tok)
    y = g.matmul_q8(x, q, s)
    xv = (np.random.default_rng(n_tok).standard_normal((n_tok, dim)) * 0.25).astype(np.float32)
    g.set_input(x, xv)
    g.execute()
    got = g.output_f32(y)
    assert got.size == n_tok * rows
    assert same_bits(got, O.Mat.q8_parts(q, s).apply(xv))


def test_attention_block():
    # runs_an_attention_block (lib.rs:264-293): seq 4, 2 heads, head_dim 8
    seq, nh, hd = 4, 2, 8
    width = nh * hd
    g = P.Graph()
    x = g.input(seq)
    wq, wk, wv = sinw(width * width, 0.001), sinw(width * width, 0.002), sinw(width * width, 0.003)
    q0, k0, v0 = g.matmul_f32(x, wq, width, width), g.matmul_f32(x, wk, width, width), g.matmul_f32(x, wv, width,
                                                                                                        width)
    q, k = g.rope(q0, nh, hd, 10000.0), g.rope(k0, nh, hd, 10000.0)
    attn = g.attention(q, k, v0, nh, nh, hd)
    out = g.add(attn, x)
    xv = np.cos(np.arange(seq * width, dtype=np.float32) * np.float32(0.02)).astype(np.float32).reshape(seq, width)
    g.set_input(x, xv)
    g.execute()
    y = g.output_f32(out)
    assert y.size == seq * width and np.isfinite(y).all()
    oq = O.rope_batch(O.Mat.f32(wq.reshape(width, width)).apply(xv), seq, nh, hd, 10000.0)
    ok = O.rope_batch(O.Mat.f32(wk.reshape(width, width)).apply(xv), seq, nh, hd, 10000.0)
    ov = O.Mat.f32(wv.reshape(width, width)).apply(xv)
    oa = O.attention(oq, ok, ov, seq, nh, nh, hd)
    assert same_bits(g.output_f32(q), oq) and same_bits(g.output_f32(k), ok)
    assert same_bits(g.output_f32(attn), oa) and same_bits(y, oa + xv)


def demo_block(g, seq, n_heads, n_kv_heads, head_dim, ffn, q8=False):
    """prana-cli demo (main.rs:276-315) built on g; returns (input id, out id,
    the oracle's output for the same input)."""
    dim = n_heads * head_dim
    kvw = n_kv_heads * head_dim

    def mat(rows, cols, seed):
        return sinw(rows * cols, seed, 0.1).reshape(rows, cols)

    ws = {"q": mat(dim, dim, 0.0011), "k": mat(kvw, dim, 0.0013), "v": mat(kvw, dim, 0.0017),
          "o": mat(dim, dim, 0.0019), "up": mat(ffn, dim, 0.0007), "down": mat(dim, ffn, 0.0009)}
    ones = np.ones(dim, np.float32)
    x = g.input(seq)
    omat = {}

    def mm(node, name):
        w = ws[name]
        if q8 and w.shape[1] % 32 == 0:
            q, s = O.quantize_q8(w)
            omat[name] = O.Mat.q8_parts(q, s)
            return g.matmul_q8(node, q, s)
        omat[name] = O.Mat.f32(w)
        return g.matmul_f32(node, w, w.shape[1], w.shape[0])

    n1 = g.rmsnorm(x, ones, dim, 1e-5)
    q0, k0, v0 = mm(n1, "q"), mm(n1, "k"), mm(n1, "v")
    q, k = g.rope(q0, n_heads, head_dim, 10000.0), g.rope(k0, n_kv_heads, head_dim, 10000.0)
    attn = g.attention(q, k, v0, n_heads, n_kv_heads, head_dim)
    res1 = g.add(mm(attn, "o"), x)
    n2 = g.rmsnorm(res1, ones, dim, 1e-5)
    out = g.add(mm(mm(n2, "up"), "down"), res1)

    xv = np.sin(np.arange(seq * dim, dtype=np.float32) * np.float32(0.01)).astype(np.float32).reshape(seq, dim)
    on1 = O.rmsnorm(xv, ones, 1e-5)
    oq = O.rope_batch(omat["q"].apply(on1), seq, n_heads, head_dim, 10000.0)
    ok = O.rope_batch(omat["k"].apply(on1), seq, n_kv_heads, head_dim, 10000.0)
    oa = O.attention(oq, ok, omat["v"].apply(on1), seq, n_heads, n_kv_heads, head_dim)
    ores1 = (omat["o"].apply(oa) + xv).astype(np.float32)
    on2 = O.rmsnorm(ores1, ones, 1e-5)
    oout = (omat["down"].apply(omat["up"].apply(on2)) + ores1).astype(np.float32)
    return x, out, xv, oout


@pytest.mark.parametrize("seq,nh,nkv,hd,ffn,q8", [(8, 4, 2, 16, 128, False), (8, 4, 2, 16, 128, True),
                                                  (300, 8, 2, 32, 512, True), (40, 6, 3, 64, 768, False)])
def test_cli_demo_block(seq, nh, nkv, hd, ffn, q8):
    g = P.Graph()
    x, out, xv, want = demo_block(g, seq, nh, nkv, hd, ffn, q8)
    g.set_input(x, xv)
    g.execute()
    y = g.output_f32(out)
    assert np.isfinite(y).all() and same_bits(y, want)


def test_unset_input_and_shape_errors():
    # unset_input_is_an_error_not_a_crash (lib.rs:296-304)
    g = P.Graph()
    x = g.input(1)
    y = g.rmsnorm(x, np.ones(4, np.float32), 4, 1e-5)
    with pytest.raises(P.GraphError) as e:
        g.execute()
    assert e.value.kind == "UnsetInput" and e.value.node == x
    with pytest.raises(P.PranaError, match="unset"):
        g.output_f32(y)
    # shape mismatches name the node
    g = P.Graph()
    a = g.input(2)
    b = g.input(2)
    mm = g.matmul_f32(a, np.ones(6, np.float32), 3, 2)   # expects 2 x 3 values
    s = g.add(a, b)
    g.set_input(a, np.ones(8, np.float32), (2, 4))
    g.set_input(b, np.ones(8, np.float32), (2, 4))
    with pytest.raises(P.GraphError) as e:
        g.execute()
    assert e.value.kind == "ShapeMismatch" and e.value.node == mm and "matmul_f32 input" in str(e.value)
    g2 = P.Graph()
    a, b = g2.input(1), g2.input(1)
    s = g2.add(a, b)
    r = g2.rope(a, 2, 2, 1e4)
    g2.set_input(a, np.ones(4, np.float32))
    g2.set_input(b, np.ones(3, np.float32))
    with pytest.raises(P.GraphError) as e:
        g2.execute()
    assert e.value.kind == "ShapeMismatch" and e.value.node == s and "add" in str(e.value)
    # ids are checked when a node is built
    with pytest.raises(P.PranaError, match="does not exist"):
        g2.add(a, 99)
    with pytest.raises(P.PranaError, match="even"):
        g2.rope(a, 1, 3, 1e4)
    with pytest.raises(P.PranaError, match="multiple of n_kv_heads"):
        g2.attention(a, a, a, 3, 2, 4)
    assert r > s


def test_values_are_cached_reset_recomputes_and_device_inputs():
    dim = 64
    g = P.Graph()
    x = g.input(3)
    w = sinw(dim * dim, 0.003).reshape(dim, dim)
    y = g.matmul_f32(x, w, dim, dim)
    z = g.softmax(y)
    x1 = np.random.default_rng(1).standard_normal((3, dim)).astype(np.float32)
    x2 = np.random.default_rng(2).standard_normal((3, dim)).astype(np.float32)
    g.set_input(x, x1)
    g.execute()
    first = g.output_f32(z)
    # execute keeps computed values (lib.rs:132-141): a new input alone changes nothing
    g.set_input(x, x2)
    g.execute()
    assert same_bits(g.output_f32(z), first)
    # reset drops them; the inputs stay
    g.reset()
    g.execute()
    m = O.Mat.f32(w)
    assert same_bits(g.output_f32(y), m.apply(x2)) and same_bits(g.output_f32(z), O.softmax(m.apply(x2).ravel()))
    # an input from device memory
    d = P.DeviceArray.from_host(x1)
    g.set_input(x, d)
    g.reset()
    g.execute()
    assert same_bits(g.output_f32(z), first)
    d.free()
    # set_input on a computed node: execute keeps the given value downstream
    g2 = P.Graph()
    a = g2.input(1)
    b = g2.matmul_f32(a, np.ones(4, np.float32), 2, 2)
    c = g2.add(b, a)
    g2.set_input(a, np.float32([1, 2]), (1, 2))
    g2.set_input(b, np.float32([10, 20]), (1, 2))
    g2.execute()
    assert g2.output_f32(c).tolist() == [11.0, 22.0]
