"""CPU: graph-level fusion detection (ggml_hip_moe_fusion_detect) on hand-built
node lists of MoE FFN blocks, through the product's host code linked against the
simulated device (device / host memory kinds come from the simulated allocator).

The patterns are the ones ggml-cuda's graph evaluator fuses ahead of the
reference's intercept (patches/apply_patches.py:42-62; the fusion arguments are
consumed at kernels/moe-cache.cu:109-129): up MUL_MAT_ID [-> MUL scale] [-> ADD_ID
bias], the same for the gate, a GLU over both, and a shared expert's MUL_MATs + GLU
on the same activations (moe-cache.cu:103-106, :148-152)."""
import ctypes as C

import pytest

F32, I32 = 0, 26


class Graph:
    """Builds ggml_hip_moe_node arrays with fresh simulated buffers."""

    def __init__(self, mc, sim, *, wtype=None, K=256, R=64, n_exp=8, n_used=4, n_tok=1):
        self.mc, self.sim = mc, sim
        self.wtype = mc.Q4_K if wtype is None else wtype
        self.K, self.R, self.n_exp, self.n_used, self.n_tok = K, R, n_exp, n_used, n_tok
        self.nodes = []
        self.keep = []
        self.x = self.f32([K, 1, n_tok], self.dev(4 * K * n_tok))
        self.ids = self.tensor(I32, [n_used, n_tok], [4, 4 * n_used], self.dev(4 * n_used * n_tok))

    # memory
    def dev(self, n):
        p = self.sim.mc_sim_dev_alloc(n)
        assert p
        return p

    def host(self, n):
        p = self.sim.mc_sim_host_alloc(n)
        assert p
        return p

    # tensors
    def tensor(self, typ, ne, nb, data):
        t = self.mc.Tensor()
        t.type = typ
        ne = list(ne) + [1] * (4 - len(ne))
        nb = list(nb)
        while len(nb) < 4:
            nb.append(nb[-1] * ne[len(nb) - 1])
        t.ne[:] = ne
        t.nb[:] = nb
        t.data = data
        t.has_buffer = 1
        return t

    def f32(self, ne, data=None):
        nb = [4]
        for k in range(1, len(ne)):
            nb.append(nb[-1] * ne[k - 1])
        return self.tensor(F32, ne, nb, data if data is not None else self.dev(4 * _prod(ne)))

    def weights(self, n_exp=None, host=False, wtype=None, rows=None, name="w"):
        n_exp = self.n_exp if n_exp is None else n_exp
        wt = self.wtype if wtype is None else wtype
        rows = self.R if rows is None else rows
        nbytes = self.mc.row_bytes(wt, self.K) * rows * n_exp
        p = self.host(nbytes) if host else self.dev(nbytes)
        return self.mc.make_tensor(wt, self.K, rows, n_exp, p, name=name, keep=self.keep)

    # nodes
    def add(self, op, t, srcs, glu_op=0, glu_limit=0.0, swapped=0):
        n = self.mc.Node()
        n.op = op
        n.t = t
        for k in range(3):
            s = srcs[k] if k < len(srcs) else None
            if s is None:
                n.src[k] = -1
            elif isinstance(s, int):
                n.src[k] = s
            else:
                n.src[k] = -1
                n.leaf[k] = s
        n.glu_op, n.glu_limit, n.glu_swapped = glu_op, glu_limit, swapped
        self.nodes.append(n)
        return len(self.nodes) - 1

    def expert_path(self, w, *, scale=None, bias=None, x=None, ids=None):
        """MUL_MAT_ID [-> MUL(scale)] [-> ADD_ID(bias)]; returns (first, last) node indices."""
        mc = self.mc
        out = self.f32([self.R, self.n_used, self.n_tok])
        x = self.x if x is None else x
        ids = self.ids if ids is None else ids
        first = cur = self.add(mc.OP_MUL_MAT_ID, out, [w, x, ids])
        if scale is not None:
            cur = self.add(mc.OP_MUL, self.f32([self.R, self.n_used, self.n_tok]), [cur, scale, ids])
        if bias is not None:
            cur = self.add(mc.OP_ADD_ID, self.f32([self.R, self.n_used, self.n_tok]), [cur, bias, ids])
        return first, cur

    def glu(self, gate, up, op, swapped=0, limit=0.0):
        srcs = [up, gate] if swapped else [gate, up]
        return self.add(self.mc.OP_GLU, self.f32([self.R, self.n_used, self.n_tok]), srcs, glu_op=op,
                        glu_limit=limit, swapped=swapped)

    def shared(self, op, host=False, wtype=None, rows=None, x=None):
        mc = self.mc
        rows = self.R if rows is None else rows
        xs = x if x is not None else self.f32([self.K, self.n_tok], self.x.data)
        wu = self.weights(1, host=host, wtype=wtype, rows=rows, name="sh_up")
        wg = self.weights(1, host=host, wtype=wtype, rows=rows, name="sh_gate")
        u = self.add(mc.OP_MUL_MAT, self.f32([rows, self.n_tok]), [wu, xs])
        g = self.add(mc.OP_MUL_MAT, self.f32([rows, self.n_tok]), [wg, xs])
        out = self.f32([rows, self.n_tok])
        k = self.add(mc.OP_GLU, out, [g, u], glu_op=op)
        return u, g, k, wu, wg, out

    def bias(self, stride=None):
        stride = self.R if stride is None else stride
        return self.tensor(F32, [self.R, self.n_exp], [4, 4 * stride], self.dev(4 * stride * self.n_exp))

    def scale(self):
        return self.tensor(F32, [1, self.n_exp], [4, 4], self.dev(4 * self.n_exp))

    def detect(self, i_up):
        return self.mc.fusion_detect(self.nodes, i_up, library=self.sim)


def _prod(xs):
    p = 1
    for x in xs:
        p *= x
    return p


def covered_set(cov):
    return {k for k, c in enumerate(cov) if c}


@pytest.fixture
def cache_off(sim, mc):
    assert sim.ggml_hip_moe_cache_reset() == 0
    cfg = mc.Config()
    cfg.enabled = 0
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    return sim


@pytest.fixture
def cache_on(sim, mc):
    assert sim.ggml_hip_moe_cache_reset() == 0
    cfg = mc.Config()
    cfg.enabled, cfg.slots, cfg.max_promotions = 1, 4, 48
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    yield sim
    assert sim.ggml_hip_moe_cache_reset() == 0


def test_plain_mul_mat_id_fuses_nothing(mc, cache_off):
    g = Graph(mc, cache_off)
    up = g.add(mc.OP_MUL_MAT_ID, g.f32([g.R, g.n_used, 1]), [g.weights(), g.x, g.ids])
    g.add(mc.OP_OTHER, g.f32([g.R, g.n_used, 1]), [up])
    n, f, gh, cov, out = g.detect(up)
    assert n == 1 and covered_set(cov) == {up} and out == up and gh is None
    assert not f.gate and not f.x_bias and not f.x_scale and not f.shared_up and f.shared_type == -1


@pytest.mark.parametrize("op", [0, 1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("swapped", [0, 1])
def test_gate_up_glu_device_weights(mc, cache_off, op, swapped):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    k = g.glu(gate, up, op, swapped=swapped, limit=7.0)
    n, f, gh, cov, out = g.detect(up)
    assert n == 3 and covered_set(cov) == {up, gate, k} and out == k
    assert f.gate == wg.data and gh is None
    assert f.glu_op == op and f.glu_limit == pytest.approx(7.0)
    assert not f.x_bias and not f.gate_bias and not f.x_scale and not f.gate_scale


def test_gate_up_order_in_graph_does_not_matter(mc, cache_off):
    """The gate MUL_MAT_ID may come first in the node array."""
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    gate, _ = g.expert_path(wg)
    up, _ = g.expert_path(wu)
    k = g.glu(gate, up, mc.GLU_SWIGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 3 and out == k and f.gate == wg.data


def test_biases_and_scales(mc, cache_off):
    """MUL_MAT_ID -> MUL(scale[ids]) -> ADD_ID(bias[ids]) on both paths, bias rows with a padded stride."""
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    xb, gb, xs, gs = g.bias(stride=g.R + 16), g.bias(stride=g.R + 16), g.scale(), g.scale()
    up, up_end = g.expert_path(wu, scale=xs, bias=xb)
    gate, gate_end = g.expert_path(wg, scale=gs, bias=gb)
    k = g.glu(gate_end, up_end, mc.GLU_SWIGLU_OAI, limit=7.0)
    n, f, gh, cov, out = g.detect(up)
    assert n == 7 and covered_set(cov) == {up, up + 1, up + 2, gate, gate + 1, gate + 2, k} and out == k
    assert f.x_bias == xb.data and f.gate_bias == gb.data and f.bias_stride == g.R + 16
    assert f.x_scale == xs.data and f.gate_scale == gs.data and f.gate == wg.data


def test_bias_only_on_one_path(mc, cache_off):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    gb = g.bias()
    up, up_end = g.expert_path(wu)
    gate, gate_end = g.expert_path(wg, bias=gb)
    k = g.glu(gate_end, up_end, mc.GLU_GEGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 4 and out == k and f.gate_bias == gb.data and not f.x_bias and f.bias_stride == g.R


def test_mismatched_bias_strides_are_not_fused(mc, cache_off):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, up_end = g.expert_path(wu, bias=g.bias(stride=g.R))
    gate, gate_end = g.expert_path(wg, bias=g.bias(stride=g.R + 8))
    g.glu(gate_end, up_end, mc.GLU_SWIGLU)
    n, f, gh, cov, out = g.detect(up)
    # the GLU cannot take two strides; the up path's own bias still fuses into the GEMV
    assert not f.gate and out == up_end and covered_set(cov) == {up, up + 1} and f.x_bias


def test_bias_after_scale_order_only(mc, cache_off):
    """ADD_ID before MUL computes (w.x + b) * s, which the kernel's scale-then-bias epilogue does not:
    the MUL is left to the graph."""
    g = Graph(mc, cache_off)
    wu = g.weights(name="up")
    xb, xs = g.bias(), g.scale()
    up = g.add(mc.OP_MUL_MAT_ID, g.f32([g.R, g.n_used, 1]), [wu, g.x, g.ids])
    a = g.add(mc.OP_ADD_ID, g.f32([g.R, g.n_used, 1]), [up, xb, g.ids])
    m = g.add(mc.OP_MUL, g.f32([g.R, g.n_used, 1]), [a, xs, g.ids])
    n, f, gh, cov, out = g.detect(up)
    assert out == a and covered_set(cov) == {up, a} and f.x_bias == xb.data and not f.x_scale
    assert not cov[m]


def test_up_path_alone_fuses_bias_and_scale(mc, cache_off):
    g = Graph(mc, cache_off)
    wu = g.weights(name="up")
    xb, xs = g.bias(), g.scale()
    up, up_end = g.expert_path(wu, scale=xs, bias=xb)
    g.add(mc.OP_OTHER, g.f32([g.R, g.n_used, 1]), [up_end])
    n, f, gh, cov, out = g.detect(up)
    assert n == 3 and out == up_end and f.x_bias == xb.data and f.x_scale == xs.data and not f.gate


def test_extra_consumer_blocks_fusion(mc, cache_off):
    """An intermediate read by another node must be materialised: nothing past it fuses."""
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    g.glu(gate, up, mc.GLU_SWIGLU)
    g.add(mc.OP_OTHER, g.f32([g.R, g.n_used, 1]), [gate])          # the gate result is also read here
    n, f, gh, cov, out = g.detect(up)
    assert n == 1 and out == up and not f.gate
    g2 = Graph(mc, cache_off)
    wu, wg = g2.weights(name="up"), g2.weights(name="gate")
    xb = g2.bias()
    up, up_end = g2.expert_path(wu, bias=xb)
    gate, _ = g2.expert_path(wg)
    g2.glu(gate, up_end, mc.GLU_SWIGLU)
    g2.add(mc.OP_OTHER, g2.f32([g2.R, g2.n_used, 1]), [up])         # the raw up product is read elsewhere
    n, f, gh, cov, out = g2.detect(up)
    assert n == 1 and out == up and not f.x_bias and not f.gate


def test_gate_on_other_activations_or_ids(mc, cache_off):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    other_x = g.f32([g.K, 1, 1])
    gate, _ = g.expert_path(wg, x=other_x)
    g.glu(gate, up, mc.GLU_SWIGLU)
    assert g.detect(up)[4] == up
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    other_ids = g.tensor(I32, [g.n_used, 1], [4, 4 * g.n_used], g.dev(4 * g.n_used))
    gate, _ = g.expert_path(wg, ids=other_ids)
    g.glu(gate, up, mc.GLU_SWIGLU)
    assert g.detect(up)[4] == up


def test_gate_type_or_shape_mismatch(mc, cache_off):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate", wtype=mc.Q2_K)
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    g.glu(gate, up, mc.GLU_SWIGLU)
    assert g.detect(up)[4] == up
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate", n_exp=g.n_exp * 2)
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    g.glu(gate, up, mc.GLU_SWIGLU)
    assert g.detect(up)[4] == up


def test_up_as_gate_operand_is_not_fused(mc, cache_off):
    """GLU(up, gate) with swapped = 0 puts the up product in the gate slot: not the pattern."""
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    g.add(mc.OP_GLU, g.f32([g.R, g.n_used, 1]), [up, gate], glu_op=mc.GLU_SWIGLU)
    assert g.detect(up)[4] == up
    # detected from the other MUL_MAT_ID it is the ordinary pattern with roles exchanged
    n, f, gh, cov, out = g.detect(gate)
    assert n == 3 and f.gate == wu.data


def test_host_gate_without_cache_is_not_fused(mc, cache_off):
    """With the cache off the gate must be device memory the kernel reads directly."""
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate", host=True)
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    g.glu(gate, up, mc.GLU_SWIGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 1 and not f.gate and gh is None


def test_cache_path_gate_goes_to_gate_host(mc, cache_on):
    """Host-resident experts the cache wants: the gate is handed over as a tensor (its own table)."""
    g = Graph(mc, cache_on)
    wu, wg = g.weights(name="up", host=True), g.weights(name="gate", host=True)
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    k = g.glu(gate, up, mc.GLU_SWIGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 3 and out == k and not f.gate
    assert gh is not None and gh.data == wg.data and gh.type == wg.type and list(gh.ne) == list(wg.ne)


def test_shared_expert(mc, cache_off):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    k = g.glu(gate, up, mc.GLU_SWIGLU)
    su, sg, sk, swu, swg, sout = g.shared(mc.GLU_SWIGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 6 and covered_set(cov) == {up, gate, k, su, sg, sk} and out == k
    assert f.shared_up == swu.data and f.shared_gate == swg.data and f.shared_type == swu.type
    assert f.shared_dst == sout.data and f.shared_stride_col_dst == g.R


def test_shared_expert_without_routed_gate(mc, cache_off):
    """A shared GLU fuses beside a plain up GEMV too; its GLU op becomes the launch's."""
    g = Graph(mc, cache_off)
    up, _ = g.expert_path(g.weights(name="up"))
    su, sg, sk, swu, swg, sout = g.shared(mc.GLU_GEGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 4 and out == up and f.shared_up == swu.data and f.glu_op == mc.GLU_GEGLU and not f.gate


@pytest.mark.parametrize("case", ["host", "glu_op", "rows", "type", "other_x", "batch"])
def test_shared_expert_negatives(mc, cache_off, case):
    g = Graph(mc, cache_off)
    wu, wg = g.weights(name="up"), g.weights(name="gate")
    up, _ = g.expert_path(wu)
    gate, _ = g.expert_path(wg)
    g.glu(gate, up, mc.GLU_SWIGLU)
    if case == "host":
        g.shared(mc.GLU_SWIGLU, host=True)
    elif case == "glu_op":
        g.shared(mc.GLU_GEGLU)                     # one GLU op per launch
    elif case == "rows":
        g.shared(mc.GLU_SWIGLU, rows=g.R * 2)      # the shared row blocks are the routed ones
    elif case == "type":
        g.shared(mc.GLU_SWIGLU, wtype=mc.Q8_1)      # not a weight type
    elif case == "other_x":
        g.shared(mc.GLU_SWIGLU, x=g.f32([g.K, 1]))
    elif case == "batch":
        ws = g.weights(2, name="sh_batched")
        xs = g.f32([g.K, 1], g.x.data)
        u = g.add(mc.OP_MUL_MAT, g.f32([g.R, 1]), [ws, xs])
        gg = g.add(mc.OP_MUL_MAT, g.f32([g.R, 1]), [ws, xs])
        g.add(mc.OP_GLU, g.f32([g.R, 1]), [gg, u], glu_op=mc.GLU_SWIGLU)
    n, f, gh, cov, out = g.detect(up)
    assert n == 3 and not f.shared_up and f.shared_type == -1


def test_malformed_input_is_an_error(mc, cache_off):
    g = Graph(mc, cache_off)
    up = g.add(mc.OP_MUL_MAT_ID, g.f32([g.R, g.n_used, 1]), [g.weights(), g.x, g.ids])
    o = g.add(mc.OP_OTHER, g.f32([g.R, g.n_used, 1]), [up])
    with pytest.raises(mc.MoeError, match="not a MUL_MAT_ID"):
        g.detect(o)
    g.nodes[o].src[1] = 5
    with pytest.raises(mc.MoeError, match="out of range"):
        g.detect(up)
