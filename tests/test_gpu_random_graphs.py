"""Seeded random captured steps, replayed against an eager twin.

Each case builds a random step of 2 to 5 operations on one stream, chosen from
the graph-replayable entry points: the fused layer step over a device-side
position counter (a counter of its own or one shared with another layer, with
or without the position advance in the step), the batched paged layer step
over device-side positions, and the ragged decode over device-side lengths
(unit grid or stream-K).  Shapes, cache types and options are drawn too.  Two
copies of every buffer are made: the step is captured once over the first copy
and replayed for several steps; the second copy runs the same operations
eagerly.  Between steps the host writes new inputs, lengths and positions into
both copies.  A replay launches the kernels the eager calls launch, with the
same arguments, so after every step the outputs, caches, page pools and
counters of the two copies must be equal bit for bit; the first and last
steps are also checked against the oracle (tmac_gguf.cpp:990-1016, 1090-1091,
1093-1128): outputs to |gpu - ref| <= 2e-5 + 1e-4 |ref|, written cache rows bit
for bit.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close
from test_gpu_random_more import reset_options, set_options
from test_gpu_random_shapes import DTYPES, PR, SHAPES, paged_pool, pool_rows, store, widen

pytestmark = pytest.mark.gpu
HD = 64


class Twin:
    """One logical buffer held twice (graph copy, eager copy)."""

    def __init__(self, ctx, host):
        self.g = ctx.upload(np.ascontiguousarray(host))
        self.e = ctx.upload(np.ascontiguousarray(host))

    def write(self, host, stream):
        self.g.copy_from(host, stream=stream)
        self.e.copy_from(host, stream=stream)

    def pick(self, eager):
        return self.e if eager else self.g

    def same(self, what, stream):
        a, b = self.g.numpy(stream=stream), self.e.numpy(stream=stream)
        np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8), err_msg=what)
        return a

    def free(self):
        self.g.free()
        self.e.free()


@pytest.mark.parametrize("seed", range(24))
def test_random_step_graph_matches_eager(ctx, seed):
    rng = np.random.default_rng(12000 + seed)
    g, kv = SHAPES[int(rng.integers(len(SHAPES)))]
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    nh, kvd = g * kv, kv * HD
    n_ops = int(rng.integers(2, 6))
    steps = 5
    opts = dict(kernel=int(rng.integers(0, 4)), mfma=int(rng.integers(0, 2)), stream_k=int(rng.choice([0, 1, 2])))
    set_options(ctx, **opts)
    s = ctx.stream()
    twins, ops = [], []

    def twin(host):
        t = Twin(ctx, host)
        twins.append(t)
        return t

    kinds = []
    try:
        cap = 64 + int(rng.integers(0, 64))
        counters = [twin(np.array([int(rng.integers(0, 40))], np.int32)) for _ in range(2)]
        for i in range(n_ops):
            kind = ["layer", "layer", "paged_layer", "ragged"][int(rng.integers(4))]
            kinds.append(kind)
            if kind == "layer":
                c = int(rng.integers(2))
                kc = twin(store(oracle.normal(12100 + 10 * seed + i, (cap, kvd)), dt, kv))
                vc = twin(store(oracle.normal(12200 + 10 * seed + i, (cap, kvd)), dt, kv))
                op = dict(kind=kind, c=c, kc=kc, vc=vc, q=twin(np.zeros(nh * HD, np.float32)),
                          kn=twin(np.zeros(kvd, np.float32)), vn=twin(np.zeros(kvd, np.float32)),
                          out=twin(np.zeros(nh * HD, np.float32)))
            elif kind == "paged_layer":
                n_seq = int(rng.integers(1, 4))
                max_len = 48 + 16 * int(rng.integers(0, 4))
                max_pages = (max_len + PR - 1) // PR
                n_pages = n_seq * max_pages + 2
                rows = [store(oracle.normal(12300 + 10 * seed + 5 * i + q, (max_len, kvd)), dt, kv)
                        for q in range(n_seq)]
                kp, table = paged_pool(rows, n_pages, np.random.default_rng(12400 + seed + i))
                vrows = [store(oracle.normal(12500 + 10 * seed + 5 * i + q, (max_len, kvd)), dt, kv)
                         for q in range(n_seq)]
                vp, _ = paged_pool(vrows, n_pages, np.random.default_rng(12400 + seed + i))
                op = dict(kind=kind, n_seq=n_seq, max_len=max_len, n_pages=n_pages, table=table,
                          tab=twin(table), kp=twin(kp), vp=twin(vp),
                          pos=twin(rng.integers(0, max_len - steps, n_seq).astype(np.int32)),
                          q=twin(np.zeros((n_seq, nh * HD), np.float32)),
                          kn=twin(np.zeros((n_seq, kvd), np.float32)), vn=twin(np.zeros((n_seq, kvd), np.float32)),
                          out=twin(np.zeros((n_seq, nh * HD), np.float32)))
            else:
                n_seq = int(rng.integers(1, 6))
                max_len = int(rng.integers(16, 700))
                offs = (np.arange(n_seq) * max_len).astype(np.int64)
                k = store(oracle.normal(12600 + 10 * seed + i, (n_seq * max_len, kvd)), dt, kv)
                v = store(oracle.normal(12700 + 10 * seed + i, (n_seq * max_len, kvd)), dt, kv)
                op = dict(kind=kind, n_seq=n_seq, max_len=max_len, offs=offs, k=twin(k), v=twin(v),
                          doffs=twin(offs), lens=twin(np.full(n_seq, max_len, np.int32)),
                          q=twin(np.zeros((n_seq, nh * HD), np.float32)),
                          out=twin(np.zeros((n_seq, nh * HD), np.float32)))
            ops.append(op)
        advance = [bool(rng.integers(0, 2)), bool(rng.integers(0, 2))]
        what = f"seed {seed}: g={g} kv={kv} dt={dt} ops={kinds} advance={advance} {opts}"
        ctx.rope_prepare(HD, 1e6, cap + 64)

        def run(eager):
            for op in ops:
                P = lambda name: op[name].pick(eager)  # noqa: E731
                if op["kind"] == "layer":
                    ctx.layer_attention_devpos(P("q"), P("kn"), P("vn"), P("kc"), P("vc"), P("out"), nh, kv, HD,
                                               counters[op["c"]].pick(eager), cap, 1e6, stream=s, kv_dtype=dt)
                elif op["kind"] == "paged_layer":
                    ctx.layer_attention_paged(P("q"), P("kn"), P("vn"), P("kp"), P("vp"), op["n_pages"], P("tab"),
                                              op["table"].shape[1], P("pos"), P("out"), op["n_seq"], nh, kv, HD,
                                              op["max_len"], 1e6, stream=s, kv_dtype=dt)
                else:
                    ctx.decode_ragged(P("q"), P("k"), P("v"), P("doffs"), P("lens"), P("out"), op["n_seq"], nh, kv,
                                      HD, op["max_len"], stream=s, kv_dtype=dt)
            for c, adv in zip(counters, advance):
                if adv:
                    ctx.pos_update(c.pick(eager), 1, add=True, stream=s)

        run(False)  # one eager pass over each copy first: workspace and tables are
        run(True)  # sized before the capture, and both copies stay equal
        ctx.synchronize(s)
        ctx.step_begin(s)
        run(False)
        graph = ctx.step_end(s)
        try:
            for step in range(steps):
                for i, op in enumerate(ops):
                    base = 13000 + 100 * seed + 10 * step + i
                    op["q"].write(oracle.normal(base, op["q"].g.shape), s)
                    if op["kind"] in ("layer", "paged_layer"):
                        op["kn"].write(oracle.normal(base + 1, op["kn"].g.shape), s)
                        op["vn"].write(oracle.normal(base + 2, op["vn"].g.shape), s)
                    if op["kind"] == "paged_layer":
                        pos = op["pos"].g.numpy(stream=s)
                        op["pos"].write(np.minimum(pos + 1, op["max_len"] - 1).astype(np.int32), s)
                    if op["kind"] == "ragged":
                        op["lens"].write(rng.integers(0, op["max_len"] + 1, op["n_seq"]).astype(np.int32), s)
                start = []
                for c in counters:  # keep both counters inside the cache
                    p = int(c.g.numpy(stream=s)[0])
                    if p >= cap - 1:
                        p = 0
                        c.write(np.zeros(1, np.int32), s)
                    start.append(p)
                ctx.graph_launch(graph, s)
                run(True)
                ctx.synchronize(s)
                for t_i, t in enumerate(twins):
                    t.same(f"{what} step {step} buffer {t_i}", s)
                if step in (0, steps - 1):
                    check_oracle(ops, nh, kv, dt, start, s, what + f" step {step}")
        finally:
            ctx.graph_destroy(graph)
    finally:
        reset_options(ctx)
        ctx.synchronize(s)
        for t in twins:
            t.free()
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


def check_oracle(ops, nh, kv, dt, start, s, what):
    """Every operation of the step just run against the oracle, on the eager
    copy (equal to the graph copy by then).  start[c] is counter c's value when
    the step began: the position every fused layer step on that counter used."""
    for op in ops:
        got = op["out"].e.numpy(stream=s)
        q = op["q"].e.numpy(stream=s)
        if op["kind"] == "ragged":
            lens = op["lens"].e.numpy(stream=s)
            nz = lens > 0
            assert np.all(got[~nz] == 0), what
            if nz.any():
                k = widen(op["k"].e.numpy(stream=s), dt, kv)
                v = widen(op["v"].e.numpy(stream=s), dt, kv)
                ref = oracle.attention_ragged(q[nz], k, v, op["offs"][nz], lens[nz], nh, kv, HD, n_threads=8)
                assert_close(got[nz], ref, what + " ragged")
            continue
        kn, vn = op["kn"].e.numpy(stream=s), op["vn"].e.numpy(stream=s)
        if op["kind"] == "layer":
            p = start[op["c"]]
            kc, vc = op["kc"].e.numpy(stream=s), op["vc"].e.numpy(stream=s)
            qr, kr = oracle.rope(q, kn, nh, kv, HD, p, 1e6)
            np.testing.assert_array_equal(kc[p], store(kr, dt, kv)[0], err_msg=what + " layer k row")
            np.testing.assert_array_equal(vc[p], store(vn, dt, kv)[0], err_msg=what + " layer v row")
            ref = oracle.attention(qr, widen(kc[:p + 1], dt, kv), widen(vc[:p + 1], dt, kv), nh, kv, HD, p)
            assert_close(got, ref, what + f" layer pos {p}")
            continue
        pos = op["pos"].e.numpy(stream=s)
        kp, vp = op["kp"].e.numpy(stream=s), op["vp"].e.numpy(stream=s)
        for sq in range(op["n_seq"]):
            p = int(pos[sq])
            qr, kr = oracle.rope(q[sq], kn[sq], nh, kv, HD, p, 1e6)
            rows = pool_rows(op["table"], sq, p + 1)
            np.testing.assert_array_equal(kp[rows[-1]], store(kr, dt, kv)[0], err_msg=what + " paged k row")
            np.testing.assert_array_equal(vp[rows[-1]], store(vn[sq], dt, kv)[0], err_msg=what + " paged v row")
            ref = oracle.attention(qr, widen(kp[rows], dt, kv), widen(vp[rows], dt, kv), nh, kv, HD, p)
            assert_close(got[sq], ref, what + f" paged layer seq {sq} pos {p}")
