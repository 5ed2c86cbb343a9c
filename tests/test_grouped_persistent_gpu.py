"""The persistent grouped W4A16 launch (lhq_gemm_w4a16_bf16_grouped_ws and
its SwiGLU form, the grouped contract of gemm.cpp:69-75 over the
expert_offsets table of moe.cpp:111-123).

One launch of P = 2 x CUs workgroups walks the (group, 64-row tile,
256-column group) tiles counted from the device-side table, tile t on
workgroup t % P; when the T tiles fill at most three quarters of one round
(T <= 3P/4) and the workspace holds the segments, they are spread along K
over all workgroups instead (stream-K), their fp32 partial sums added in K
order by a fixup kernel.  `_plan` restates that choice so each case asserts
which path it covers.

Every case checks the GPU output against the oracle (gemm_quant.cpp:54-82
per group, asymmetric int4 codes with fp16 scales and u4 zeros, bf16
activations; relative Frobenius <= 1e-2 and > 99% of elements within one
bf16 ulp), on every row and all columns, or a sample of columns where N is
large (the weight format is per column, so the oracle on the sliced codes is
exact).  The split changes only fp32 summation order, so the output does not
depend on the workspace's prior contents and repeats bit for bit."""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu

TOL_BF16 = 1e-2
SLOT = 64 * 1024  # bytes of one tile's partial sums


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _workers():
    import torch
    return 2 * torch.cuda.get_device_properties(0).multi_processor_count


def _plan(rows_per_group, Nt, Kt, slots):
    """(T, q, R, stream-K?) of the persistent launch for this table."""
    P = _workers()
    X = -(-Nt // 16)
    T = X * sum(-(-r // 64) for r in rows_per_group)
    q, R = divmod(T, P)
    Ps = min(P, max(1, R * Kt // 4))
    sk = q == 0 and R > 0 and 4 * R <= 3 * P and Ps + R - 1 <= slots  # slots: 1 where T_max rules it out
    return T, q, R, sk


def _codes(oracle, g, K, N, G):
    p = g.integers(0, 256, (K // 2, N), dtype=np.uint8)
    s = oracle.f32_to_f16_n(g.uniform(0.0005, 0.004, (K // G, N)).astype(np.float32))
    z = g.integers(0, 16, (K // G, N), dtype=np.uint8)
    return p, s, z


def _check(oracle, got, want, exact_want=False):
    err = rel_frobenius(got, want)
    assert err <= TOL_BF16, err
    want_b = want if exact_want else D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want))
    assert (np.abs(got - want_b) <= np.abs(want_b) * 2.0 ** -7 + 1e-30).mean() > 0.99


class Case:
    """A grouped problem: bf16 activations for rows_per_group rows per group,
    random per-group codes, its prepacked weights and pointer tables."""

    def __init__(self, oracle, ops, rows_per_group, K, N, G, seed, swiglu=False):
        self.off = np.concatenate([[0], np.cumsum(rows_per_group)]).astype(np.int32)
        self.rows_per_group, self.K, self.N, self.G, self.swiglu = list(rows_per_group), K, N, G, swiglu
        self.rows = int(self.off[-1])
        g = D.rng(seed)
        self.A = D.to_bf16_bits(oracle, g.standard_normal((self.rows, K)).astype(np.float32))
        E = len(rows_per_group)
        self.codes = [_codes(oracle, g, K, N, G) for _ in range(E)]
        if swiglu:
            self.up = [_codes(oracle, g, K, N, G) for _ in range(E)]
            Ws = []
            for c, u in zip(self.codes, self.up):
                wg = ops.prepack_w4_asym(*(ops.dev(a) for a in c), K, N, G)
                wu = ops.prepack_w4_asym(*(ops.dev(a) for a in u), K, N, G)
                Ws.append(ops.interleave_gate_up(wg, wu))
        else:
            Ws = [ops.prepack_w4_asym(*(ops.dev(a) for a in c), K, N, G) for c in self.codes]
        self.Ws = Ws
        self.tables = ops.pointer_tables(Ws)
        self.cols = np.arange(N) if N <= 512 else np.unique(np.concatenate(
            [np.arange(16), np.arange(N - 16, N), g.choice(N, 48, replace=False)]))

    @property
    def Nt(self):
        nt = -(-self.N // 16)
        return 2 * nt if self.swiglu else nt

    def workspace_bytes(self, ops):
        fn = ("lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes" if self.swiglu
              else "lhq_gemm_w4a16_bf16_grouped_workspace_bytes")
        return getattr(ops.lib().cdll, fn)(len(self.rows_per_group), self.rows, self.N, self.K, self.G)

    def run(self, ops, ws=None, ws_bytes=0):
        q, s, z = self.tables
        C = ops.zeros((self.rows, self.N), np.int16)
        E = len(self.rows_per_group)
        print(f"grouped{'_swiglu' if self.swiglu else ''} rows={self.rows_per_group} K={self.K} N={self.N} "
              f"G={self.G} ws={ws_bytes}", flush=True)
        if ws is None:
            name = "lhq_gemm_w4a16_bf16_grouped_swiglu" if self.swiglu else "lhq_gemm_w4a16_bf16_grouped"
            ops.run(name, self.A, self.off, q, s, z, C, E, self.rows, self.N, self.K, self.G)
        else:
            name = "lhq_gemm_w4a16_bf16_grouped_swiglu_ws" if self.swiglu else "lhq_gemm_w4a16_bf16_grouped_ws"
            ops.run(name, self.A, self.off, q, s, z, C, E, self.rows, self.N, self.K, self.G, ws, ws_bytes)
        return ops.host(C, np.uint16)

    def want(self, oracle):
        cols = self.cols
        sl = lambda c: [np.ascontiguousarray(a[:, cols]) for a in c]  # noqa: E731
        out = np.zeros((self.rows, len(cols)), np.float32)
        for e in range(len(self.rows_per_group)):
            lo, hi = int(self.off[e]), int(self.off[e + 1])
            if hi == lo:
                continue
            v = oracle.gemm_w4a16_asym(self.A[lo:hi], *sl(self.codes[e]), len(cols), self.G)
            if self.swiglu:
                u = oracle.gemm_w4a16_asym(self.A[lo:hi], *sl(self.up[e]), len(cols), self.G)
                v = D.bf16_bits_to_f32(oracle.swiglu_bf16(v, u))
            out[lo:hi] = v
        return out

    def check(self, oracle, out):
        _check(oracle, D.bf16_bits_to_f32(out[:, self.cols]), self.want(oracle), exact_want=self.swiglu)


def _workspace(ops, nbytes, fill=None):
    import torch
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    if fill is not None:
        ws.fill_(fill)
    return ws


# (rows per group, K, N, G): each case names the path it covers on MI355X's
# 256 CUs (P = 512 workers); _plan asserts it on the box it runs on.
CASES = {
    # config 4 routing at reduced N: T = 20 tiles < P, all split (4 K tiles
    # per worker, eight segments per tile)
    "all_split": ([123, 115, 133, 136, 114, 147, 134, 122], 4096, 256, 128),
    # T = 1 x 15 tiles, Kt = 2: parts of 4-5 K tiles hold whole tiles
    # (stream-K workers that write whole tiles as well as segments)
    "whole_tiles_in_split": ([100, 200, 50, 300, 170], 256, 200, 128),
    # ragged table: empty groups, 1-row and 64 / 65-row groups, N % 16 != 0
    "ragged": ([0, 1, 63, 64, 65, 130, 0, 200], 1024, 3000, 128),
    # G = 384 (group index by multiply-high): 4-tile parts cut groups of 3
    "g384": ([90, 150, 70, 260], 1536, 520, 384),
    # 70 groups of 50-70 rows: the table resolves in two steps of 64 groups
    "many_groups": (list(np.random.default_rng(7).integers(50, 71, 70)), 1024, 256, 128),
    # T = 8 x 64 = 512 = P: one round of whole tiles
    "exact_round": ([512] * 8, 256, 2048, 128),
    # T = 9 x 100 = 900: whole tiles, a second round on 388 workgroups
    "two_rounds": ([640] * 10, 256, 2304, 128),
    # T = 9 x 64 = 576: a second round of 64 tiles, Kt = 8
    "round_and_64": ([512] * 8, 1024, 2304, 128),
    # T = 7 x 64 = 448 > 3P/4: one round of whole tiles, nothing split
    "most_of_a_round": ([512] * 8, 256, 1792, 128),
}


@pytest.mark.parametrize("name", list(CASES))
def test_grouped_persistent_matches_oracle(oracle, ops, name):
    rows, K, N, G = CASES[name]
    c = Case(oracle, ops, rows, K, N, G, seed=100 + list(CASES).index(name))
    need = c.workspace_bytes(ops)
    assert need > 0 and need % SLOT == 0
    T, q, R, sk = _plan(rows, c.Nt, K // 128, need // SLOT)
    if _workers() == 512:
        expect = {"all_split": (0, True), "whole_tiles_in_split": (0, True), "ragged": (0, True),
                  "g384": (0, True), "many_groups": (0, True), "exact_round": (1, False),
                  "two_rounds": (1, False), "round_and_64": (1, False), "most_of_a_round": (0, False)}[name]
        assert (q, sk) == expect, (T, q, R, sk)
    ws = _workspace(ops, need, fill=0x7F)  # any contents
    out = c.run(ops, ws, need)
    c.check(oracle, out)


def test_grouped_persistent_repeats_and_ignores_workspace_contents(oracle, ops):
    c = Case(oracle, ops, [123, 115, 133, 136, 114, 147, 134, 122], 2048, 512, 128, seed=9)
    need = c.workspace_bytes(ops)
    a = c.run(ops, _workspace(ops, need, fill=0), need)
    b = c.run(ops, _workspace(ops, need, fill=0xFF), need)  # NaN bit patterns
    assert np.array_equal(a, b)
    assert np.array_equal(a, c.run(ops, _workspace(ops, need, fill=0x41), need))
    c.check(oracle, a)


def test_grouped_persistent_small_workspace_and_none(oracle, ops):
    """A workspace of one slot cannot hold the split: the persistent launch
    deals every tile whole.  No workspace: the one-workgroup-per-tile grid."""
    c = Case(oracle, ops, [200, 90, 300], 1024, 768, 128, seed=12)
    T, q, R, sk = _plan(c.rows_per_group, c.Nt, 8, 1)
    assert not sk
    one = c.run(ops, _workspace(ops, SLOT), SLOT)
    c.check(oracle, one)
    none = c.run(ops)
    c.check(oracle, none)
    full = c.run(ops, _workspace(ops, c.workspace_bytes(ops)), c.workspace_bytes(ops))
    c.check(oracle, full)
    # whole tiles run the same K loop: bit-identical to the grid launch
    assert np.array_equal(one, none)


@pytest.mark.parametrize("rows,K,I", [
    ([123, 115, 133, 136, 114, 147, 134, 122], 1024, 256),   # T = 2 x 20 = 40: all split
    ([300, 0, 41, 270], 512, 1000),                          # ragged, I % 16 != 0
])
def test_grouped_swiglu_persistent(oracle, ops, rows, K, I):
    c = Case(oracle, ops, rows, K, I, 128, seed=31, swiglu=True)
    need = c.workspace_bytes(ops)
    assert need > 0
    out = c.run(ops, _workspace(ops, need, fill=0x55), need)
    c.check(oracle, out)


def test_grouped_workspace_bytes(ops):
    P = _workers()
    L = ops.lib().cdll
    # a few rows per group: the 16-row kernel, no workspace
    assert L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(8, 16, 4096, 4096, 128) == 0
    # the tile kernel: P + T_max - 1 slots, T_max = X (ceil(rows / 64) + live groups), where
    # T_max <= 3P/4 allows a split; one slot (the persistent launch alone) otherwise
    assert L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(8, 1024, 256, 4096, 128) == (P + 24 - 1) * SLOT
    assert L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(8, 1024, 14336, 4096, 128) == SLOT
    # config 4's down projection: T_max = 16 x 24 = 384 = 3P/4 at P = 512
    if P == 512:
        assert L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(8, 1024, 4096, 14336, 128) == (P + 384 - 1) * SLOT
    # the SwiGLU form counts 2 ceil(I / 16) column tiles
    assert (L.lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes(8, 1024, 200, 4096, 128)
            == (P + 2 * 24 - 1) * SLOT)
    # G < 128 runs no tile kernel
    assert L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(8, 1024, 14336, 4096, 64) == 0
    assert L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(0, 1024, 14336, 4096, 128) == 0


def test_grouped_ws_rejects_misaligned_workspace(ops):
    import torch
    from longhornai_amd import capi
    c_off = torch.tensor([0, 64, 128], dtype=torch.int32, device="cuda")
    ws = torch.empty(2 * SLOT + 64, dtype=torch.uint8, device="cuda")
    L = ops.lib().cdll
    dummy = torch.zeros(1, dtype=torch.int64, device="cuda")
    A = torch.zeros((128, 256), dtype=torch.int16, device="cuda")
    C = torch.zeros((128, 256), dtype=torch.int16, device="cuda")
    st = L.lhq_gemm_w4a16_bf16_grouped_ws(A.data_ptr(), c_off.data_ptr(), dummy.data_ptr(), dummy.data_ptr(),
                                          dummy.data_ptr(), C.data_ptr(), 2, 128, 256, 256, 128,
                                          ws.data_ptr() + 4, 2 * SLOT, None)
    assert st == capi.LHQ_ERR_INVALID
    assert "aligned" in ops.lib().last_error()


def test_expert_mlp_ws_matches_oracle(oracle, ops):
    """lhq_moe_expert_mlp_w4a16_bf16_ws: the SwiGLU and down launches of the
    expert MLP (moe.cpp:150-196) sharing one workspace."""
    import torch
    rows = [123, 115, 133, 136, 114, 147, 134, 122]
    H, I, G = 512, 768, 128
    gu = Case(oracle, ops, rows, H, I, G, seed=61, swiglu=True)
    dn_codes = [_codes(oracle, D.rng(62 + e), I, H, G) for e in range(len(rows))]
    dn = [ops.prepack_w4_asym(*(ops.dev(a) for a in c), I, H, G) for c in dn_codes]
    dq, ds, dz = ops.pointer_tables(dn)
    q, s, z = gu.tables
    L = ops.lib().cdll
    need = max(L.lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes(8, gu.rows, I, H, G),
               L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(8, gu.rows, H, I, G))
    assert need > 0
    ws = _workspace(ops, need, fill=0x33)
    act = ops.zeros((gu.rows, I), np.int16)
    y = ops.zeros((gu.rows, H), np.int16)
    ops.run("lhq_moe_expert_mlp_w4a16_bf16_ws", gu.A, gu.off, q, s, z, dq, ds, dz, act, y, 8, gu.rows, H, I, G,
            ws, need)
    act_h = ops.host(act, np.uint16)
    y_h = D.bf16_bits_to_f32(ops.host(y, np.uint16))
    gu.check(oracle, act_h)
    want = np.zeros((gu.rows, H), np.float32)
    for e in range(8):
        lo, hi = int(gu.off[e]), int(gu.off[e + 1])
        want[lo:hi] = oracle.gemm_w4a16_asym(act_h[lo:hi], *dn_codes[e], H, G)
    _check(oracle, y_h, want)
    # the same as the two calls without a workspace, within the bf16 bar
    act2 = ops.zeros((gu.rows, I), np.int16)
    y2 = ops.zeros((gu.rows, H), np.int16)
    ops.run("lhq_moe_expert_mlp_w4a16_bf16", gu.A, gu.off, q, s, z, dq, ds, dz, act2, y2, 8, gu.rows, H, I, G)
    assert rel_frobenius(D.bf16_bits_to_f32(ops.host(y2, np.uint16)), y_h) <= TOL_BF16
    del dn, gu
    torch.cuda.empty_cache()


@pytest.mark.parametrize("rows,K,N", [
    ([123, 115, 133, 136, 114, 147, 134, 122], 2048, 256),    # split along K: tile kernel + fixup
    ([512] * 8, 256, 2048),                                   # one round of whole tiles
])
def test_grouped_persistent_in_a_captured_hip_graph(oracle, ops, rows, K, N):
    """The persistent launch (and its fixup) allocates nothing and records no
    memset, so it can be captured: a graph of one call is replayed three
    times with new activations written into its input and the output
    cleared eagerly between replays; each replay equals the eager call on
    the same input bit for bit."""
    import torch
    c = Case(oracle, ops, rows, K, N, 128, seed=77)
    n = c.workspace_bytes(ops)
    ws = _workspace(ops, n)
    A = ops.dev(c.A)
    off = ops.dev(c.off)
    q, s, z = c.tables
    C = ops.zeros((c.rows, N), np.int16)
    E = len(rows)
    L = ops.lib().cdll

    def call():
        st = L.lhq_gemm_w4a16_bf16_grouped_ws(A.data_ptr(), off.data_ptr(), q.data_ptr(), s.data_ptr(),
                                              z.data_ptr(), C.data_ptr(), E, c.rows, N, K, 128, ws.data_ptr(), n,
                                              ops.stream())
        assert st == 0, ops.lib().last_error()

    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            call()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for rep in range(3):
        A.copy_(ops.dev(D.to_bf16_bits(oracle, D.rng(200 + rep).standard_normal((c.rows, K)).astype(np.float32))))
        C.zero_()
        call()
        want = ops.host(C, np.uint16).copy()
        C.zero_()
        g.replay()
        torch.cuda.synchronize()
        print(f"grouped graph replay {rep}", flush=True)
        assert np.array_equal(ops.host(C, np.uint16), want), f"replay {rep}"
