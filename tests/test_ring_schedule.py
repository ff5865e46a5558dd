"""CPU replay of the hand-counted memory waits of the kernels that stage operands through LDS with
buffer->LDS requests (kern_amd/csrc/kern_mx.hip): the GEMM ring (ring_prologue / ring_kloop / the chained
tiles of bmm_moe, and bmm_tile) and the row-group GEMVs.

Such a request writes LDS asynchronously, and the compiler does not track it: every read of the data waits
for it by hand, with `s_waitcnt vmcnt(n)` (at most n of this wave's vector-memory operations still
outstanding; they retire in issue order) and, when other waves read it, a workgroup barrier after that wait.
Each wave's program is written out here as the kernel issues it (requests, the other vector-memory
operations the counts include -- epilogue stores, route_map loads, weight loads into registers --, waits,
barriers, LDS reads and the points where the read data is consumed), and a checker proves on the host:

* read after write: every LDS read finds the data it expects (tile, k-tile) in every piece it reads, the
  request that wrote it retired by a wait of its issuing wave that happens before the read (same wave: in
  program order; another wave: a barrier in between);
* write after read: no request that overwrites a piece is issued before every read of the piece's earlier
  data has completed (the reading wave consumed it, or waited for LDS, before a barrier that precedes the
  request);
* every request has retired when the wave ends, and all waves pass the same number of barriers.

The checker is exercised on a planted mistake (a count one too large, a missing barrier, a refill one
barrier early) so that it is known to catch each kind, and on a reconstruction of the GEMV variant that
staged x by buffer->LDS requests one k-tile ahead with a fixed count (the form dropped after one sweep
mismatch): the last k-tile of every wave has fewer weight requests behind its x request than the fixed
count assumes.
"""
import itertools

import pytest

# ------------------------------------------------------------------------------------------ the checker


def _hb(a, b):
    """Point a = (wave, epoch, pos) happens before point b: same wave in program order, or a barrier between."""
    return a[1] < b[1] if a[0] != b[0] else a[2] < b[2]


def check(programs):
    """Replay per-wave programs; raise AssertionError naming the first hazard. Ops:
    ("req", piece, content)  buffer->LDS request (counts in vmcnt)
    ("vm",)                  any other vector-memory operation (counts in vmcnt)
    ("wait", n)              s_waitcnt vmcnt(n)
    ("bar",)                 workgroup barrier
    ("read", piece, content) LDS read expecting `content` in `piece`
    ("done",)                the wave's earlier LDS reads have completed (lgkmcnt(0), or their data consumed)"""
    writes, reads, bars = {}, [], []
    for w, prog in enumerate(programs):
        epoch, out, pending = 0, [], []
        for pos, op in enumerate(prog):
            k = op[0]
            if k == "req":
                rec = {"at": (w, epoch, pos), "piece": op[1], "content": op[2], "done": None}
                writes.setdefault(op[1], []).append(rec)
                out.append(rec)
            elif k == "vm":
                out.append(None)
            elif k == "wait":
                while len(out) > op[1]:
                    r = out.pop(0)
                    if r is not None:
                        r["done"] = (w, epoch, pos)
            elif k == "bar":
                epoch += 1
            elif k == "read":
                rec = {"at": (w, epoch, pos), "piece": op[1], "content": op[2], "done": None}
                reads.append(rec)
                pending.append(rec)
            elif k == "done":
                for r in pending:
                    r["done"] = (w, epoch, pos)
                pending = []
            else:
                raise ValueError(op)
        assert all(r is None for r in out), f"wave {w}: requests into LDS outstanding at the end"
        for r in pending:  # reads never consumed: complete at the wave's end
            r["done"] = (w, epoch, len(prog))
        bars.append(epoch)
    assert len(set(bars)) == 1, f"waves pass different numbers of barriers: {bars}"
    for wr in writes.values():
        owners = {r["at"][0] for r in wr}
        assert len(owners) == 1, f"piece {wr[0]['piece']} written by several waves {owners}"
    for rd in reads:
        wr = writes.get(rd["piece"], [])
        seen = [i for i, r in enumerate(wr) if r["done"] is not None and _hb(r["done"], rd["at"])]
        assert seen, f"read of {rd['piece']} at {rd['at']} (wants {rd['content']}): no request retired before it"
        k = seen[-1]
        assert wr[k]["content"] == rd["content"], \
            f"read of {rd['piece']} at {rd['at']} wants {rd['content']}, finds {wr[k]['content']}"
        for r in wr[k + 1:]:
            if r["content"] != rd["content"]:
                assert _hb(rd["done"], r["at"]), (
                    f"request of {r['content']} into {rd['piece']} at {r['at']} may land before the read at "
                    f"{rd['at']} (wanting {rd['content']}) has completed")


# ------------------------------------------------------------------------------------------ the GEMM ring

FC2, FC1, PT, DENSE = "fc2", "fc1", "pt", "dense_bf16"


def epi_stores(mode):
    """Stores each wave sends in a ring tile's epilogue (kern_mx.hip epi_stores)."""
    return 2 + 4 if mode == FC1 else (4 if mode == PT else 8)


def ring_nxr(valid):
    return min(4, max(1, (valid + 31) >> 5))


def live_ts(valid, wt):
    return min(4, max(0, (valid - wt * 64 + 15) >> 4))


class Ring:
    """One workgroup's ring programs (8 waves: group 0 = waves 0-3 fill weights, group 1 = 4-7 activations)
    over a sequence of tiles with the given live-row counts, as bmm_moe (persistent, chained) or bmm_tile
    (one tile) issue them. `mistake` plants one error on the CPU to show the checker catches it."""

    def __init__(self, mode, KT, valids, persistent=True, mistake=None):
        assert KT % 4 == 0 and KT >= 4
        self.mode, self.KT, self.KG = mode, KT, KT // 4
        self.valids, self.persistent, self.mistake = valids, persistent, mistake
        self.R = 6 if (mode == FC1 and persistent) else 0
        self.ST = epi_stores(mode)

    # requests of wave gw of a group (pieces are (kind, slot or stage, index); contents (kind, tile, k))
    def req_w(self, p, gw, tile, kt, stage):
        for r in range(4):
            p.append(("req", ("W", stage, r * 4 + gw), ("w", tile, kt)))

    def req_ws(self, p, gw, tile, kg, slot):
        for r in range(4):
            p.append(("req", ("SW", slot, r * 4 + gw), ("sw", tile, kg)))

    def req_x(self, p, gw, tile, kt, stage, nxr):
        for r in range(nxr):
            p.append(("req", ("X", stage, r * 4 + gw), ("x", tile, kt)))

    def req_xs(self, p, gw, tile, kg, slot, nxr):
        for h in range(2 if nxr > 2 else 1):
            p.append(("req", ("SX", slot, 4 * h + gw), ("sx", tile, kg)))

    def read_tile(self, p, wt, wn, tile, kt, stage, with_sw, nts):
        kg, jt = kt // 4, kt % 4
        for rs in range(4):
            p.append(("read", ("W", stage, wn * 4 + rs), ("w", tile, kt)))
        if with_sw:
            for rs in range(4):
                p.append(("read", ("SW", kg & 1, wn * 4 + rs), ("sw", tile, kg)))
        for ts in range(nts):
            t0 = wt * 64 + ts * 16
            for b in (t0 >> 3, (t0 >> 3) + 1):
                p.append(("read", ("X", stage, b), ("x", tile, kt)))
            if jt == 0:
                p.append(("read", ("SX", kg & 1, t0 >> 4), ("sx", tile, kg)))

    def wave(self, w):
        wt, wn = w >> 2, w & 3
        grp, gw = wt, wn
        KT, KG, R, ST, mis = self.KT, self.KG, self.R, self.ST, self.mistake
        n = len(self.valids)
        p = []
        p += [("vm",)] * R  # ring_tile of the pass's first tile (its route_map loads)
        # ring_prologue
        v0 = self.valids[0]
        if grp == 0:
            self.req_ws(p, gw, 0, 0, 0)
            for kt in range(4):
                self.req_w(p, gw, 0, kt, kt)
        else:
            nx = ring_nxr(v0)
            self.req_xs(p, gw, 0, 0, 0, nx)
            for kt in range(3):
                self.req_x(p, gw, 0, kt, kt, nx)
        for e in range(n):
            chain = e + 1 < n
            tn = e + 1 if chain else e
            first = e == 0
            valid = self.valids[e]
            nts = live_ts(valid, wt)
            nxr = ring_nxr(valid)
            nxs = 2 if nxr > 2 else 1
            wn_kg = 0 if chain else KG - 1
            p += [("vm",)] * R  # ring_tile(Tn): its route_map loads
            # ring_kloop: the first wait
            if grp == 0:
                cnt = 12 + R if first else 12 + R + ST
            else:
                cnt = 2 * nxr + R if first else 8 + R + ST
            if mis == "first_wait_plus_one" and e == 1 and grp == 0:
                cnt += 1
            p.append(("wait", cnt))
            p.append(("bar",))
            if grp == 0:
                self.read_tile(p, wt, wn, e, 0, 0, True, nts)
                for kt in range(KT):
                    jt, kg, last = kt % 4, kt // 4, kt >= KT - 4
                    p.append(("done",))  # mfmas of tile kt consume the operands read before
                    if not last or jt < 3:
                        p.append(("wait", 8 + (4 if jt in (1, 2) else 0)))
                    if not (mis == "drop_barrier" and kt == 1):
                        p.append(("bar",))
                    if mis == "early_refill" and kt == 2:  # the refill moved before the half-step's barrier
                        p.insert(len(p) - 1, ("req", ("W", jt, gw), ("w", e, kt + 4)))
                    if not last:
                        if jt == 0:
                            self.req_ws(p, gw, e, kg + 1, (kg + 1) & 1)
                        self.req_w(p, gw, e, kt + 4, jt)
                    else:
                        if jt == 0:
                            self.req_ws(p, gw, tn, wn_kg, 0)
                        self.req_w(p, gw, tn, jt if chain else KT - 1, jt)
                    if not last or jt < 3:
                        self.read_tile(p, wt, wn, e, kt + 1, (jt + 1) & 3, jt == 3, nts)
                    p.append(("bar",))
                if mis == "drop_barrier":
                    p.append(("bar",))
            else:
                for kt in range(KT):
                    jt, kg, last = kt % 4, kt // 4, kt >= KT - 4
                    if not last or jt == 0:
                        if not last and jt == 1:
                            self.req_xs(p, gw, e, kg + 1, (kg + 1) & 1, nxr)
                        self.req_x(p, gw, e, kt + 3, (jt + 3) & 3, nxr)
                    else:
                        if jt == 1:
                            self.req_xs(p, gw, tn, wn_kg, 0, 4)
                        self.req_x(p, gw, tn, jt - 1 if chain else KT - 1, (jt + 3) & 3, 4)
                    self.read_tile(p, wt, wn, e, kt, jt, jt == 0, nts)
                    p.append(("done",))  # WAIT_LGKMCNT0
                    if not last:
                        p.append(("wait", 2 * nxr + (nxs if jt in (1, 2) else 0)))
                    elif jt < 3:
                        p.append(("wait", 2 * nxr if jt == 0 else (nxr + 6 if jt == 1 else 10)))
                    p.append(("bar",))
                    p.append(("done",))  # mfmas
                    p.append(("bar",))
            p += [("vm",)] * ST  # the epilogue's stores
        p.append(("wait", 0))  # the last tile's requests land before the LDS is used again or released
        return p

    def programs(self):
        return [self.wave(w) for w in range(8)]


# Row counts a tile can have: the loader's cases 1-32 (1 block), 33-64 (2), 65-80, 81-96 (3), 97-112, 113-128
_VALIDS = [1, 16, 17, 32, 33, 64, 65, 80, 81, 96, 97, 112, 113, 128]


@pytest.mark.parametrize("mode", [FC2, FC1])
@pytest.mark.parametrize("KT", [4, 8, 12, 28])
def test_ring_chained_tiles(mode, KT):
    """Persistent passes of up to three chained tiles over every pair of row-count cases (K = 512 .. 3584:
    one, two, three and seven k groups, both parities of the scale slots)."""
    vals = _VALIDS if KT <= 8 else [1, 17, 33, 65, 81, 97, 113, 128]
    for a, b in itertools.product(vals, repeat=2):
        check(Ring(mode, KT, [a, b]).programs())
    for vs in [[128, 17, 128], [5, 128, 64], [64, 64, 64], [100, 1, 33]]:
        check(Ring(mode, KT, vs).programs())
    for v in _VALIDS:
        check(Ring(mode, KT, [v]).programs())


@pytest.mark.parametrize("mode", [PT, DENSE])
@pytest.mark.parametrize("KT", [4, 8, 56, 64])
def test_ring_dense_tile(mode, KT):
    """bmm_tile: one tile per workgroup (first and unchained), every row-count case of a last token block."""
    for v in _VALIDS:
        check(Ring(mode, KT, [v], persistent=False).programs())


@pytest.mark.parametrize("mistake", ["first_wait_plus_one", "drop_barrier", "early_refill"])
def test_ring_checker_catches_planted_mistakes(mistake):
    with pytest.raises(AssertionError):
        check(Ring(FC1, 8, [128, 128, 128], mistake=mistake).programs())


def test_ring_without_the_epilogue_stores_in_the_count():
    """The chained tile's first wait counts the previous epilogue's stores exactly: had the first tile's
    stores not been sent (fewer vector-memory operations than counted), that wait would let the next tile's
    reads run ahead of its first requests."""
    ring = Ring(FC2, 8, [128, 128])
    progs = []
    for prog in ring.programs():
        prog = list(prog)
        stores = [i for i, op in enumerate(prog) if op == ("vm",)][: ring.ST]  # FC2 sends no other such op
        for i in reversed(stores):
            del prog[i]
        progs.append(prog)
    with pytest.raises(AssertionError):
        check(progs)


# ------------------------------------------------------------------------------------------ the GEMVs


def gemv_rows_fixed(M, NKT, D=4):
    """kern_mx_gemv_bf16_r{NKT}: per wave, x slice (M tokens x NKT*16 pieces, 64 a request) and the scale
    fragments by buffer->LDS requests, then D weight loads into registers, WAIT_VMCNT(D), then its own reads
    (each wave reads only its own region: no barrier)."""
    progs = []
    D = min(D, NKT)
    for w in range(4):
        p = []
        for t in range(M):
            for q in range(0, NKT * 16, 64):
                p.append(("req", ("xg", w, t, q), ("x", t, q)))
        p.append(("req", ("ssc", w), ("s",)))
        p += [("vm",)] * D
        p.append(("wait", D))
        p.append(("read", ("ssc", w), ("s",)))
        for i in range(NKT):
            for t in range(M):
                for q in range(0, NKT * 16, 64):
                    if i == 0:
                        p.append(("read", ("xg", w, t, q), ("x", t, q)))
            p.append(("done",))
            if i + D < NKT:
                p.append(("vm",))
        p.append(("wait", 0))
        p.append(("bar",))
        progs.append(p)
    return progs


@pytest.mark.parametrize("M,NKT", [(1, 14), (2, 14), (3, 14), (16, 4), (9, 16), (1, 2), (8, 2)])
def test_gemv_row_group_waits(M, NKT):
    check(gemv_rows_fixed(M, NKT))


def gemv_rg(M, KG):
    """kern_mx_gemv_bf16_rg: per wave, its k groups' x (one request per token and group) by buffer->LDS
    requests, then one scale load and four weight loads into registers, WAIT_VMCNT(5)."""
    progs = []
    for w in range(4):
        g0, ng = (w * KG) >> 2, (((w + 1) * KG) >> 2) - ((w * KG) >> 2)
        p = []
        for g in range(ng):
            for t in range(M):
                p.append(("req", ("xg", w, g, t), ("x", g0 + g, t)))
        if ng > 0:
            p += [("vm",)] * 5
            p.append(("wait", 5))
            for g in range(ng):
                p += [("vm",)]
                for t in range(M):
                    p.append(("read", ("xg", w, g, t), ("x", g0 + g, t)))
                p.append(("done",))
                p += [("vm",)] * 4
        p.append(("wait", 0))
        p.append(("bar",))
        progs.append(p)
    return progs


@pytest.mark.parametrize("M,KG", [(1, 1), (2, 3), (1, 7), (2, 32)])
def test_gemv_rg_waits(M, KG):
    check(gemv_rg(M, KG))


def gemv_persistent_x_by_dma(KTW, M, exact, NG=5, D=6):
    """The dropped variant of kern_mx_gemv_bf16_p{KTW}: the persistent walk (item i = j*NG + g is fragment
    (g, k-tile j); weights D items ahead, the request for item i + D sent after item i while i + D < TOT),
    with each wave's next k-tile of x sent by buffer->LDS requests into the other half of its 8 KiB (one
    request per 4 token rows that hold a present token) as k-tile j starts, and waited for by an explicit
    count before k-tile j + 1 reads it. exact=False: the count is the steady state's (NG weight requests
    behind the x requests); exact=True: the count of requests actually sent behind them."""
    TOT = NG * KTW
    nreq = (M + 3) // 4
    progs = []
    for w in range(8):
        p = []
        for q in range(nreq):
            p.append(("req", ("xst", w, 0, q), ("x", 0)))
        p += [("vm",)] * min(D, TOT)
        behind = {}  # k-tile j+1 -> weight requests sent after its x requests
        for i in range(TOT):
            g, j = i % NG, i // NG
            if g == 0:
                if j == 0:
                    p.append(("wait", min(D, TOT)))
                else:
                    n_after = behind[j]
                    p.append(("wait", n_after if exact else NG))
                for q in range(nreq):
                    p.append(("read", ("xst", w, j & 1, q), ("x", j)))
                p.append(("done",))
                if j + 1 < KTW:
                    for q in range(nreq):
                        p.append(("req", ("xst", w, (j + 1) & 1, q), ("x", j + 1)))
                    behind[j + 1] = 0
            if i + D < TOT:
                p.append(("vm",))
                if j + 1 < KTW and (j + 1) in behind:
                    behind[j + 1] += 1
        p.append(("wait", 0))
        p.append(("bar",))
        progs.append(p)
    return progs


@pytest.mark.parametrize("KTW", [1, 2, 7, 8])
def test_gemv_staged_x_variant_fixed_count_is_short(KTW):
    """The recorded mismatch (M = 15, N = 16640, K = 2048: kern_mx_gemv_bf16_p2, KTW = 2): with a fixed
    count, the last k-tile's x requests have NG - 1 weight requests behind them, not NG, so the count
    lets the read run ahead of the last request; the exact count is clean. KTW = 1 sends no x request
    after the first and is clean either way."""
    if KTW == 1:
        check(gemv_persistent_x_by_dma(KTW, 15, exact=False))
    else:
        with pytest.raises(AssertionError):
            check(gemv_persistent_x_by_dma(KTW, 15, exact=False))
    check(gemv_persistent_x_by_dma(KTW, 15, exact=True))


# ------------------------------------------------------------------------------------------ the code object


def _disassembly(fn):
    import os
    import re
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hsaco = os.path.join(root, "kern_amd", "lib", "kern_mx.hsaco")
    objdump = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "llvm-objdump")
    if not (os.path.exists(hsaco) and os.path.exists(objdump)):
        pytest.skip("needs the built code object and llvm-objdump")
    text = subprocess.run([objdump, "-d", "--mcpu=gfx950", hsaco], capture_output=True, text=True,
                          check=True).stdout
    out, on = [], False
    for line in text.splitlines():
        if line.endswith(f"<{fn}>:"):
            on = True
            continue
        if on and re.match(r"^[0-9a-f]+ <.*>:$", line):
            break
        m = re.match(r"\s*([a-z_0-9]+)\s*(.*?)\s*//\s*([0-9A-F]+):", line) if on else None
        if m:
            out.append((int(m.group(3), 16), m.group(1), m.group(2)))
    assert out, fn
    return out


@pytest.mark.parametrize("fn", ["kern_mx_bmm_fc1", "kern_mx_bmm_fc2", "kern_mx_gemm_e4m3", "kern_mx_gemm_bf16"])
def test_ring_epilogue_stores_are_never_lane_conditional(fn):
    """The replay above assumes every wave sends epi_stores stores per ring tile, as the source writes them
    (buffer stores whose range drops the rows past the tile). In the built code object no branch taken when
    no lane is active (s_cbranch_execz) jumps over a buffer store, so the compiler has not made any of them
    conditional; the lane-conditional stores it has are the debug output's and the small-slot epilogue's
    global stores, which no count includes."""
    ins = _disassembly(fn)
    at = {a: i for i, (a, _, _) in enumerate(ins)}
    stores = [i for i, (_, op, _) in enumerate(ins) if op.startswith("buffer_store")]
    assert stores, f"{fn}: no buffer stores found"
    for i, (a, op, arg) in enumerate(ins):
        if op != "s_cbranch_execz":
            continue
        off = int(arg.split()[0])
        off = off - 65536 if off >= 32768 else off  # the 16-bit signed word offset
        j = at[a + 4 + 4 * off]
        skipped = [ins[s][1] for s in stores if i < s < j]
        assert not skipped, f"{fn}: s_cbranch_execz at {a:#x} jumps over {skipped}"
