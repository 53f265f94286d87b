"""Generate sage_tile.inc: the tile loop of the Sage attention kernel as one
hand-scheduled inline-assembly statement.

The kernel (sage.hip, sage_attn_pipe) software-pipelines its 64-key tiles. In the
iteration of tile t every wave
  1. waits for its DMA of iteration t-2 and meets the other three waves of its
     work-group at the barrier (the LDS slots of K(t) and V(t-2) are then free; the
     wave's quarter of K(t+4) and V(t+2) is DMA'd into them during step 2);
  2. (block A) issues P(t-1) V(t-1) for output channels 0..63 and the first score
     MFMA of each key block of S(t+1), from operand registers the previous iteration
     prefetched, and refills the operand registers;
  3. (block B) runs the softmax of S(t) -- P(t) = e4m3(exp2(S(t) * sc + nm)) and the
     row sum over the unquantized values -- interleaved with the other P(t-1) V(t-1)
     and S(t+1) MFMAs and their LDS reads, prefetches the operands of iteration t+1,
     computes the row max of S(t+1) and from it tile t+1's running max m, exponent
     offset nm and rescale factor alpha, and rescales the row sum l (tile t+1 without
     dead keys: folded into the tail of the softmax stream; with dead keys: after
     masking them to -inf);
  4. rescales the output accumulators by alpha(t) when the running max moved at t.
After the last tile it adds P(last) V(last). The compiler does not keep such an
interleaving (its scheduler groups the MFMAs and the exponentials, and it copies and
spills values pinned to registers across separate asm statements), so the whole loop
is one asm statement with a fixed register map and instruction order. The loop body
is unrolled four times (tile t uses LDS slot t % 4, S and P buffers t % 2), so every
LDS address is a per-lane base register plus a compile-time offset; entry jumps to
the body of phase tb % 4.

Register map (all VGPRs pinned by the operand list in sage.hip):
  v[0:63]     output accumulators (4 blocks of 32 channels)
  v[64:95]    S buffer 0 (tiles t even), v[96:127] S buffer 1: [key block 0][key block 1]
  v[128:135]  P buffer 0, v[136:143] P buffer 1
  v[144:151]  K operands (2 x 4), v[152:167] V operands (2 x 8)
  v[168:183]  Q^T fragments (chunk cc in v[168 + 4cc : 171 + 4cc])
  v[184:199]  16 copies of the score bias 0x4B400000
  v[200:215]  scratch: exp / mask temporaries, partial row sums, max tree
  v216 kbase, v217 vbase0, v218 vbase1 (LDS read bases), v219 m, v220 l, v221 qs,
  v222 sc, v223 nm (of the tile being softmaxed), v224 scratch, v226 im,
  v227 lw (masking) / scratch (update), v239 / v225 alpha of tiles of parity 0 / 1,
  v[228:230] / v[232:234] tile table entries (parity of the tile),
  v236 / v231 / v237 per-lane DMA offsets of the two K ops / the V ops, v238 scratch
Tile table entry in LDS (16 bytes per tile, the first 12 read): liveness bits low,
high, K scale, 0.

Hazards the fixed order respects (the hardware does not interlock them):
  * VALU result -> MFMA operand: 2 wait states (block A starts with s_nop 2; block B
    with four VALU instructions; the drain with s_nop 2);
  * MFMA result -> VALU read: up to 19 wait states (the max tree reads each key block
    of S(t+1) 20 or more instructions after the last MFMA writing it; the
    accumulators are read by the rescale more than 60 instructions after their last
    MFMA; the loop ends with s_nop padding);
  * v_exp_f32 or op_sel-writing result -> VALU read: at least one instruction between;
  * VALU writing VCC -> v_cndmask reading it, VALU writing VGPR -> v_permlane32_swap,
    v_readfirstlane -> SALU read, SALU writing M0 -> LDS DMA: explicit s_nop;
  * an LDS read refills an operand register only after the MFMA that read it has
    issued (an MFMA reads its A/B operands when it issues);
  * LDS reads complete in order, so `s_waitcnt lgkmcnt(n)` with n = reads issued
    after the one needed is exact (every iteration ends with its reads complete).

Usage: python gen_sage_tile.py  (rewrites sage_tile.inc next to this file;
tests/test_abi.py checks that the committed file matches).
"""
from __future__ import annotations

import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "sage_tile.inc")

ACC = 0
S_BASE = (64, 96)
P_BASE = (128, 136)
KT = (144, 148)
VT = (152, 160)
Q0 = 168
BIAS = 184
X0, PS0, MX0 = 200, 208, 212
V_KBASE, V_VB0, V_VB1, V_M, V_L, V_QS, V_SC, V_NM = 216, 217, 218, 219, 220, 221, 222, 223
V_T0, V_T1, V_IM, V_LW = 224, 227, 226, 227
TAB = (228, 232)
V_LK, V_LV, V_U0 = 236, 237, 238
V_LK2 = 231            # per-lane offset of the second K op (rows 32..63: 16-byte halves swapped)
V_LV2 = 235            # per-lane offset of the second V^T op (16 channel rows further)
ALPHA = (239, 225)     # rescale factor of the tiles of parity 0 / 1

KTILE = 8192          # bytes per K or V^T tile slot
HEADROOM = 3.0        # lazy-max headroom H (log2 units)
LOG2_448 = 8.807354922057604


def v(i: int) -> str:
    return f"v{i}"


def rng(base: int, n: int) -> str:
    return f"v[{base}:{base + n - 1}]"


def s_reg(par: int, i: int) -> str:
    return v(S_BASE[par] + i)


def acc(db: int) -> str:
    return rng(ACC + 16 * db, 16)


def k_off(slot: int, kb: int, cc: int) -> int:
    """LDS offset (from the per-lane K base) of the K operand (key block kb, 32-channel
    chunk cc) of the tile in K slot `slot`."""
    return slot * KTILE + cc * 2048 + kb * 512


def v_off(slot: int, db: int) -> int:
    return slot * KTILE + db * 2048


def f32(x: float) -> str:
    return "0x%08x" % struct.unpack("<I", struct.pack("<f", x))[0]


class Block:
    """Instruction list with LDS-read bookkeeping for exact lgkmcnt waits."""

    def __init__(self, lines: list[str]):
        self.lines = lines
        self.reads: list[str] = []  # tags of LDS reads still in flight, oldest first

    def emit(self, s: str) -> None:
        self.lines.append(s)

    def read(self, tag: str, dst: int, addr: int, off: int, dwords: int = 4) -> None:
        op = "ds_read_b128" if dwords == 4 else "ds_read_b96"
        self.emit(f"{op} {rng(dst, dwords)}, {v(addr)}" + (f" offset:{off}" if off else ""))
        self.reads.append(tag)

    def read_v(self, tag: str, k: int, slot: int, db: int) -> None:
        """Both halves of V operand register set k: 32-channel block db of the V^T slot."""
        self.read(tag + "a", VT[k], V_VB0, v_off(slot, db))
        self.read(tag + "b", VT[k] + 4, V_VB1, v_off(slot, db))

    def wait_for(self, *tags: str) -> None:
        idx = [self.reads.index(t) for t in tags if t in self.reads]
        if not idx:
            return
        last = max(idx)
        self.emit(f"s_waitcnt lgkmcnt({len(self.reads) - 1 - last})")
        self.reads = self.reads[last + 1:]

    def drain(self) -> None:
        if self.reads:
            self.emit("s_waitcnt lgkmcnt(0)")
            self.reads = []


def mfma_pv(db: int, k: int, pprev: int) -> str:
    return f"v_mfma_f32_32x32x64_f8f6f4 {acc(db)}, {rng(VT[k], 8)}, {rng(pprev, 8)}, {acc(db)}"


def mfma_s(par_next: int, kb: int, k: int, cc: int) -> str:
    dst = rng(S_BASE[par_next] + 16 * kb, 16)
    src_c = rng(BIAS, 16) if cc == 0 else dst
    return f"v_mfma_i32_32x32x32_i8 {dst}, {rng(KT[k], 4)}, {rng(Q0 + 4 * cc, 4)}, {src_c}"


def max_tree(par: int) -> list[str]:
    """Row max of the 32 biased int32 scores of S buffer `par` into v226 (im): four
    max3 chains of eight scores (chains 0, 1 read key block 0, chains 2, 3 key block
    1), their max, then the two wave halves combined (after v_permlane32_swap,
    t1 = [x_lo, x_lo] and t2 = [x_hi, x_hi])."""
    s = lambda i: s_reg(par, i)
    t = [v(MX0 + j) for j in range(4)]
    ops = []
    for pair in ((0, 1), (2, 3)):  # key block 0 first, then key block 1
        for step in range(4):
            for c in pair:
                b = 8 * c
                if step == 0:
                    ops.append(f"v_max3_i32 {t[c]}, {s(b)}, {s(b + 1)}, {s(b + 2)}")
                elif step < 3:
                    ops.append(f"v_max3_i32 {t[c]}, {t[c]}, {s(b + 2 * step + 1)}, {s(b + 2 * step + 2)}")
                else:
                    ops.append(f"v_max_i32 {t[c]}, {t[c]}, {s(b + 7)}")
    ops.append(f"v_max3_i32 {t[0]}, {t[0]}, {t[1]}, {t[2]}")
    ops.append(f"v_max_i32 {t[0]}, {t[0]}, {t[3]}")
    ops.append(f"v_mov_b32 {t[1]}, {t[0]}")
    ops.append(f"v_mov_b32 {t[2]}, {t[0]}")
    ops.append("s_nop 1")  # VALU write -> v_permlane32_swap read: 2 wait states
    ops.append(f"v_permlane32_swap_b32 {t[1]}, {t[2]}")
    ops.append(f"v_max_i32 {v(V_IM)}, {t[1]}, {t[2]}")
    return ops


def mask_ops(par: int) -> list[str]:
    """Dead keys of S buffer `par` -> the bits of -inf: v227 (lw) holds this lane's 32
    liveness bits (bit i = score i); a sign-extended one-bit field selects the score
    or %[kdead] (v_bfi_b32), no lane masks needed."""
    ops = []
    for i in range(32):
        t = v(X0 + (i % 8))
        ops.append(f"v_bfe_i32 {t}, {v(V_LW)}, {i}, 1")
        ops.append(f"v_bfi_b32 {s_reg(par, i)}, {t}, {s_reg(par, i)}, %[kdead]")
    return ops


def softmax_stream(par: int) -> list[str]:
    """VALU stream of the softmax of S buffer `par` into P buffer `par`: per group g
    of four scores i = 4g..4g+3 (temporaries alternate between v200..203 and
    v204..207): F = fma into the exponent, E = exp2, C = pack to e4m3 (lo, hi halves
    of P register g), A = add into four partial sums; then l += their sum."""
    pc = P_BASE[par]
    tmp = lambda i: v(X0 + (i % 8))
    F = lambda i: f"v_fma_f32 {tmp(i)}, {s_reg(par, i)}, {v(V_SC)}, {v(V_NM)}"
    E = lambda i: f"v_exp_f32 {tmp(i)}, {tmp(i)}"

    def A(g, j):
        ps = v(PS0 + j)
        return f"v_add_f32 {ps}, 0, {tmp(4 * g + j)}" if g == 0 else f"v_add_f32 {ps}, {ps}, {tmp(4 * g + j)}"

    def C(g, hi):
        i = 4 * g + 2 * hi
        return f"v_cvt_pk_fp8_f32 {v(pc + g)}, {tmp(i)}, {tmp(i + 1)}" + (" op_sel:[0,0,1]" if hi else "")

    out = [F(i) for i in range(4)]
    for g in range(8):
        for j in range(4):
            out.append(E(4 * g + j))
            if g < 7:
                out.append(F(4 * (g + 1) + j))
        out += [C(g, 0), A(g, 0), A(g, 1), C(g, 1), A(g, 2), A(g, 3)]
    out += [f"v_add_f32 {v(PS0)}, {v(PS0)}, {v(PS0 + 1)}", f"v_add_f32 {v(PS0 + 2)}, {v(PS0 + 2)}, {v(PS0 + 3)}",
            f"v_add_f32 {v(PS0)}, {v(PS0)}, {v(PS0 + 2)}", f"v_add_f32 {v(V_L)}, {v(V_L)}, {v(PS0)}"]
    return out


def mid_ops(par_next: int) -> list[str]:
    """Running max and exponent offset of tile t+1 (parity par_next) from its row max
    v226 and its K scale (table entry of tile t+1):
      sc = max(qs * ks, 1e-30); c2 = 12582912 sc; tmax = im_f * sc - c2
      mnew = tmax > m + H ? tmax : m; nm = (log2 448 - H - max(mnew, -3e38)) - c2
      alpha = mnew != m ? 2^(m - mnew) : 1 (into ALPHA[par_next], the rescale of the
      accumulators after P(t) V(t)); pend[par_next] = any lane moved.
    The caller follows them with l_rescale once l holds the sum of tile t."""
    tab = TAB[par_next]
    u0, t0, t1, al = v(V_U0), v(V_T0), v(V_T1), v(ALPHA[par_next])
    return [
        f"v_mul_f32 {v(V_SC)}, {v(V_QS)}, |{v(tab + 2)}|",                 # |ks|: the sign flags dead keys
        f"v_max_f32 {v(V_SC)}, {f32(1e-30)}, {v(V_SC)}",
        f"v_mul_f32 {u0}, {f32(12582912.0)}, {v(V_SC)}",                     # c2
        f"v_fma_f32 {t0}, {v(V_IM)}, {v(V_SC)}, -{u0}",                        # tmax
        f"v_add_f32 {t1}, {f32(HEADROOM)}, {v(V_M)}",
        f"v_cmp_gt_f32 vcc, {t0}, {t1}",
        "s_nop 1",
        f"v_cndmask_b32 {t0}, {v(V_M)}, {t0}, vcc",                             # mnew
        f"v_max_f32 {t1}, {f32(-3.0e38)}, {t0}",
        f"v_sub_f32 {t1}, {f32(LOG2_448 - HEADROOM)}, {t1}",
        f"v_sub_f32 {v(V_NM)}, {t1}, {u0}",                                     # nm
        f"v_cmp_neq_f32 vcc, {t0}, {v(V_M)}",
        f"v_sub_f32 {al}, {v(V_M)}, {t0}",
        f"s_mov_b64 %[pend{par_next}], vcc",
        f"v_exp_f32 {al}, {al}",
        f"v_mov_b32 {v(V_M)}, {t0}",
        f"v_cndmask_b32 {al}, 1.0, {al}, vcc",                                 # alpha
    ]


def l_rescale(par_next: int) -> str:
    """l *= alpha of tile t+1 (after l has taken tile t's sum)."""
    return f"v_mul_f32 {v(V_L)}, {v(V_L)}, {v(ALPHA[par_next])}"


# DMA variants of an iteration (tile t, last = the unit's last tile):
#   "A": t + 4 <= last, DMAs K(t+4) and V(t+2) (4 ops);
#   "B": t + 2 <= last < t + 4, DMAs V(t+2) only (2 ops);
#   "C": last < t + 2, no DMA.
# Tiles past the last are never loaded (their slots keep older, finite bytes: K is
# int8, and V slots past the last are never read), so no load is in flight when the
# unit ends. Each body ends by waiting until at most its own DMA ops are in flight,
# i.e. for the ops of the previous iteration (the wait for iteration t-2's tiles at
# the top of iteration t).
NOPS = {"A": 4, "B": 2, "C": 0}


def iteration(k: int, var: str) -> list[str]:
    """Body of an iteration whose tile t satisfies t % 4 == k (SGPR %[t] holds t), DMA
    variant `var`. On entry v222 / v223 hold sc / nm of tile t and ALPHA[t % 2] /
    pend[t % 2] its rescale factor; on exit the same for tile t+1."""
    L: list[str] = []
    b = Block(L)
    par, nxt = k & 1, (k & 1) ^ 1
    pprev = P_BASE[nxt]
    ks1 = (k + 1) % 4       # K slot of tile t+1
    ks2 = (k + 2) % 4       # K slot of tile t+2
    vs_prev = (k + 3) % 4   # V slot of tile t-1
    vs_cur = k              # V slot of tile t
    tab_next = TAB[nxt]
    b.emit(f"sage_{var}{k}_%=:")
    # 1. the barrier: every wave's DMA of iteration t-2 landed (each waited at the end
    #    of iteration t-1), and the slots of K(t) and V(t-2) are free
    b.emit("s_barrier")
    # table entry of tile t+1 (liveness bits for the max of S(t+1), K scale for its
    # exponent, its sign set when some key is dead); %[tabp] = its LDS address
    b.emit(f"v_mov_b32 {v(V_U0)}, %[tabp]")
    b.emit("s_add_u32 %[tabp], %[tabp], 16")
    b.read("TAB", tab_next, V_U0, 0, dwords=3)
    # 2. the softmax stream of S(t) with all twelve MFMAs of the iteration spread through
    #    it (one every seven stream instructions): the score MFMAs of S(t+1) first (their
    #    results feed the max tree at the end), the P(t-1) V(t-1) MFMAs between them
    valu = softmax_stream(par)
    mf = [  # (MFMA, reads it needs, reads issued two instructions after it)
        (mfma_s(nxt, 0, 0, 0), (), [("K01", "k", 0, 1)]),
        (mfma_s(nxt, 1, 1, 0), (), [("K11", "k", 1, 1)]),
        (mfma_pv(0, 0, pprev), (), [("V2", "vp", 0, 2)]),
        (mfma_s(nxt, 0, 0, 1), ("K01",), [("K02", "k", 0, 2)]),
        (mfma_s(nxt, 1, 1, 1), ("K11",), [("K12", "k", 1, 2)]),
        (mfma_pv(1, 1, pprev), (), [("V3", "vp", 1, 3)]),
        (mfma_s(nxt, 0, 0, 2), ("K02",), [("K03", "k", 0, 3)]),
        (mfma_s(nxt, 1, 1, 2), ("K12",), [("K13", "k", 1, 3)]),
        (mfma_s(nxt, 0, 0, 3), ("K03",), [("NK0", "n", 0, 0)]),   # K(t+2) chunk 0 for the next iteration
        (mfma_s(nxt, 1, 1, 3), ("K13",), [("NK1", "n", 1, 0)]),
        (mfma_pv(2, 0, pprev), ("V2a", "V2b"), [("N0", "v", 0, 0)]),  # V(t) block 0 for the next iteration
        (mfma_pv(3, 1, pprev), ("V3a", "V3b"), [("N1", "v", 1, 1)]),  # V(t) block 1
    ]
    pos = [3 + 7 * i for i in range(len(mf))]
    s_last = (pos[8], pos[9])  # the last MFMA writing key block 0 / 1 of S(t+1)
    # this wave's DMA ops of K(t+4) -> slot k and V(t+2) -> slot (k+2)%4, one after
    # every ~20 stream instructions (a burst of them right after the barrier makes the
    # work-group's waves queue behind each other): the two K ops fill rows 0..31 and
    # 32..63 of d-chunk w (the second 4096 bytes further in memory, 1 KB further in LDS,
    # 16-byte halves swapped: per-lane offset v231), the two V^T ops channel rows
    # 32w..32w+15 and +16 (per-lane offsets v237, v235). %[kso] / %[vso] hold the
    # scalar offsets of this iteration's tiles; M0 (the LDS destination) is written one
    # stream instruction before the load that reads it.
    def dma_k(q):
        return ([f"s_add_u32 m0, %[kdm0], {k * KTILE + q * 1024}"],
                [f"buffer_load_dwordx4 {v(V_LK2 if q else V_LK)}, %[rk], %[kso] offen lds"])

    def dma_v(q):
        return ([f"s_add_u32 m0, %[vdm0], {ks2 * KTILE + q * 1024}"],
                [f"buffer_load_dwordx4 {v(V_LV2 if q else V_LV)}, %[rv], %[vso] offen lds"])

    dma_at = {}
    if var == "A":
        for at, (m0, ld) in ((6, dma_k(0)), (48, dma_k(1))):
            dma_at.setdefault(at, []).extend(m0)
            dma_at.setdefault(at + 1, []).extend(ld)
    if var in ("A", "B"):
        for at, (m0, ld) in ((27, dma_v(0)), (69, dma_v(1))):
            dma_at.setdefault(at, []).extend(m0)
            dma_at.setdefault(at + 1, []).extend(ld)

    def do_read(r):
        tag, kind, kk, x = r
        if kind == "v":     # V(t) 32-channel block x for the next iteration
            b.read_v(tag, kk, vs_cur, x)
        elif kind == "vp":  # V(t-1) 32-channel block x
            b.read_v(tag, kk, vs_prev, x)
        elif kind == "k":   # K(t+1) chunk x
            b.read(tag, KT[kk], V_KBASE, k_off(ks1, kk, x))
        else:               # K(t+2) chunk 0 for the next iteration
            b.read(tag, KT[kk], V_KBASE, k_off(ks2, kk, 0))

    # FULL (tile t+1 has no dead key): the max tree of S(t+1) and the running-max
    # update of tile t+1 go into the tail of the stream, one op after every stream op
    # from `mx_at` (the first 8 max ops read key block 0 of S(t+1), the rest key block 1);
    # the update's writes of sc / nm / l come after the stream's last use of them.
    mx_at = max(s_last[0] + 20, pos[-1] + 2)
    flag_at = mx_at - 8  # the table entry's K-scale word -> SGPR, well before the branch
    n = kq = 0
    issue: dict[int, list] = {}
    for ins in valu[:mx_at]:
        b.emit(ins)
        n += 1
        for r in issue.pop(n, []):
            do_read(r)
        for x in dma_at.pop(n, []):
            b.emit(x)
        if n == flag_at:
            b.wait_for("TAB")
            b.emit(f"v_readfirstlane_b32 %[s0], {v(tab_next + 2)}")
        if kq < len(mf) and n == pos[kq]:
            text, needs, after = mf[kq]
            b.wait_for(*needs)
            b.emit(text)
            issue.setdefault(n + 2, []).extend(after)
            kq += 1
    assert kq == len(mf) and not issue and not dma_at, (kq, issue, dma_at)
    tail = valu[mx_at:]
    # tile t+1 with a dead key (sign of its K-scale word) -> PART tail, else FULL tail.
    # Variant C may run the unit's last iteration, which has no tile t+1: its update
    # must leave m, l and alpha alone, so it takes the PART path with every key dead
    # (row max -inf: m does not move)
    if var == "C":
        b.emit("s_add_u32 %[s2], %[t], 1")
        b.emit("s_cmp_lt_i32 %[s2], %[nt]")
        b.emit("s_cselect_b32 %[s0], %[s0], -1")
    b.emit("s_cmp_lt_i32 %[s0], 0")
    b.emit(f"s_cbranch_scc1 sage_part{var}{k}_%=")
    # FULL: the max ops go one after each stream op; the update ops follow the max tree
    # and the stream's last use of sc / nm (fma) and write of l (the tile's row sum)
    xs, ys = max_tree(nxt), mid_ops(nxt)
    last_dep = max([j for j, x in enumerate(tail) if v(V_SC) in x or v(V_NM) in x], default=-1)
    full_tail, xi, yi = [], 0, 0
    for j, op in enumerate(tail):
        full_tail.append(op)
        if xi < len(xs):
            full_tail.append(xs[xi])
            xi += 1
        elif j >= last_dep and yi < len(ys):
            full_tail.append(ys[yi])
            yi += 1
    full_tail += xs[xi:] + ys[yi:] + [l_rescale(nxt)]
    assert full_tail.index(l_rescale(nxt)) > full_tail.index(f"v_add_f32 {v(V_L)}, {v(V_L)}, {v(PS0)}")
    # hazard check: first read of each key block of S(t+1) after the MFMA writing it
    kb0 = {s_reg(nxt, j) for j in range(16)}
    kb1 = {s_reg(nxt, 16 + j) for j in range(16)}
    srcs = lambda x: {y.strip() for y in x.split(None, 1)[1].split(",")[1:]} if " " in x else set()
    stream = valu[:mx_at] + full_tail
    first0 = min(i for i, x in enumerate(stream) if srcs(x) & kb0)
    first1 = min(i for i, x in enumerate(stream) if srcs(x) & kb1)
    assert first0 + 1 - s_last[0] >= 20 and first1 + 1 - s_last[1] >= 20, (first0, first1, pos)
    L.extend(full_tail)
    b.emit(f"s_branch sage_join{var}{k}_%=")
    b.emit(f"sage_part{var}{k}_%=:")
    L.extend(tail)
    assert len(valu) - s_last[1] >= 20
    # this lane's word: keys 32h .. 32h+31 (%[hmask]: lanes 32..63)
    b.emit(f"v_cndmask_b32 {v(V_LW)}, {v(tab_next)}, {v(tab_next + 1)}, %[hmask]")
    if var == "C":
        b.emit("s_cmp_lt_i32 %[s2], %[nt]")
        b.emit(f"s_cbranch_scc1 sage_live{var}{k}_%=")
        b.emit(f"v_mov_b32 {v(V_LW)}, 0")
        b.emit(f"sage_live{var}{k}_%=:")
    L.extend(mask_ops(nxt))
    L.extend(max_tree(nxt))
    L.extend(mid_ops(nxt))
    L.append(l_rescale(nxt))
    b.emit(f"sage_join{var}{k}_%=:")
    b.drain()
    # 4. rescale of the accumulators by alpha(t) when the running max moved at tile t
    #    (P(t-1) V(t-1), issued in blocks A and B, completed long before)
    b.emit(f"s_cmp_eq_u64 %[pend{par}], 0")
    b.emit(f"s_cbranch_scc1 sage_norescale{var}{k}_%=")
    for r in range(64):
        b.emit(f"v_mul_f32 {v(ACC + r)}, {v(ALPHA[par])}, {v(ACC + r)}")
    b.emit(f"sage_norescale{var}{k}_%=:")
    # this iteration's DMA ops may stay in flight; the previous iteration's have landed
    b.emit(f"s_waitcnt vmcnt({NOPS[var]})")
    # next tile: advance the scalar DMA offsets, then the variant of tile t+1
    b.emit("s_add_u32 %[t], %[t], 1")
    k1 = (k + 1) % 4
    if var == "A":
        b.emit(f"s_add_u32 %[kso], %[kso], {KTILE}")
        b.emit("s_add_u32 %[vso], %[vso], 64")
        b.emit("s_cmp_ge_i32 %[t], %[klim]")
        b.emit(f"s_cbranch_scc1 sage_B{k1}_%=")
    elif var == "B":
        b.emit("s_add_u32 %[vso], %[vso], 64")
        b.emit("s_cmp_ge_i32 %[t], %[vlim]")
        b.emit(f"s_cbranch_scc1 sage_C{k1}_%=")
    else:
        b.emit("s_cmp_ge_i32 %[t], %[nt]")
        b.emit(f"s_cbranch_scc1 sage_drain{k}_%=")
    if k == 3:
        b.emit(f"s_branch sage_{var}0_%=")
    return L


def drain(k: int) -> list[str]:
    """After the last iteration (tile t, t % 4 == k): P(t) V(t). V channel blocks 0, 1
    were prefetched into the V registers, blocks 2 and 3 are read from slot k."""
    L: list[str] = []
    b = Block(L)
    p = P_BASE[k & 1]
    b.emit(f"sage_drain{k}_%=:")
    b.emit("s_nop 2")
    b.emit(mfma_pv(0, 0, p))
    b.emit(mfma_pv(1, 1, p))
    b.read_v("V2", 0, k, 2)
    b.read_v("V3", 1, k, 3)
    b.wait_for("V2a", "V2b")
    b.emit(mfma_pv(2, 0, p))
    b.wait_for("V3a", "V3b")
    b.emit(mfma_pv(3, 1, p))
    b.emit("s_branch sage_end_%=")
    return L


def loop() -> list[str]:
    """Entry: the variant of tile t (%[klim] = last - 3, %[vlim] = last - 1), then its
    slot phase t % 4."""
    L = ["s_mov_b32 %[m0save], m0", "s_and_b32 %[s0], %[t], 3",
         "s_cmp_ge_i32 %[t], %[vlim]", "s_cbranch_scc1 sage_entryC_%=",
         "s_cmp_ge_i32 %[t], %[klim]", "s_cbranch_scc1 sage_entryB_%="]
    for var in "ABC":
        if var != "A":
            L.append(f"sage_entry{var}_%=:")
        for k in (1, 2, 3):
            L += [f"s_cmp_eq_u32 %[s0], {k}", f"s_cbranch_scc1 sage_{var}{k}_%="]
        L.append(f"s_branch sage_{var}0_%=")
    for var in "ABC":
        for k in range(4):
            L += iteration(k, var)
    for k in range(4):
        L += drain(k)
    L += ["sage_end_%=:", "s_mov_b32 m0, %[m0save]"]
    L += ["s_nop 7"] * 3  # MFMA results -> the caller's VALU reads: up to 19 wait states
    return L


def generate() -> str:
    lines = loop()
    out = ["// Generated by gen_sage_tile.py: the tile loop of sage_attn_pipe (sage.hip) as one",
           "// inline-assembly statement. Do not edit; change the generator and rerun it.", "#pragma once", "",
           "#define SAGE_TILE_LOOP \\"]
    out += [f'  "{l}\\n" \\' for l in lines]
    out += ['  ""', ""]
    return "\n".join(out)


if __name__ == "__main__":
    with open(OUT, "w") as f:
        f.write(generate())
    print(OUT)
