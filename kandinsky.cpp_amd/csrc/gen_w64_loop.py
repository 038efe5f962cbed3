#!/usr/bin/env python3
"""Writes kd_fa_w64_loop.inc: the key loop of fa_fwd_w64 (64 query rows per
wave, one wave per SIMD) as inline-asm strings, one per operand type, from
the Q fragments in LDS to O / l stored as whole lines; and
kd_fa_xlong64_loop.inc: fa_fwd_xlong64's per-unit block, the same loop for
one unit of a persistent workgroup with the next unit's Q and first K / V
tiles brought in during it.

The loop is scheduled by hand because its two ingredients need registers
that the compiler does not give it: O (64 rows x 128 floats per wave = 128
accumulation registers) and Q (64 registers) stay in AGPRs as MFMA
operands, and the softmax of one tile runs between the matrix products of
another tile of the same wave.  Per 64-key tile t (step t):

  phase 1   MFMA  S(t+1) = K(t+1) Q^T       32 x 32x32x16, K fragments from LDS
            VALU  softmax of S(t), keys 32-63   (exp2, round to T, row sums)
  check     a row whose weight sum left [0, cap]: exact max, rescale, redo
            (cap 2^64 for BF16, 2^15 for F16: every rounded weight stays finite);
            its dependent chain (moves, lane swap, add, compare) spread over
            the last MFMAs of phase 1, the branch after the last one
  phase 2   MFMA  O^T += V(t)^T P(t)^T       32 x 32x32x16, V^T by ds_read_b64_tr_b16
            VALU  softmax of S(t+1), keys 0-31

After the last tile, the epilogue: l summed over the lane pair, 1 / l by
the correctly rounded division sequence, O / l staged per 32 rows and 32
columns over the K / V tiles and stored 8 rows x 128 bytes per instruction
through a buffer resource that ends at the last valid row.

A partial last tile (Lk not a multiple of 64) runs in the loop like the
others: its K and V rows past Lk read zeros (the buffer resources end at key
Lk - 1), and in the step that computes its scores S(n-1) a block taken only
there sets the scores of keys >= Lk to -inf before any softmax reads them,
so those keys get weight 0 and never raise a row's max -- as the 32-row
kernel's tail step gives them.

Every arithmetic step is the one the 32-row kernel (kd_fa_kernel.hip)
performs, in the same order per row -- the same MFMA accumulation order over
k-steps and key steps, the same fma / exp2 / rounding, the same row sums
(the F32 weights of each 16-key step added in order, the steps combined as
(s0 + s1) + (s2 + s3)), the
same lazy-max rule (a row's running max moves, to its exact tile max, only
when the row's own weight sum leaves [0, cap]) -- so the two kernels give
bitwise identical results.

The generator also enforces the issue rules of the code it writes: wait
states between an MFMA result and its non-MFMA readers, VALU results and
MFMA or permlane readers, transcendental results and their readers, dot2
results and their readers (the hardware does not hold back a dependent
instruction there: without them the reader sees the value from before the
dot2), M0 and the LDS DMA that reads it; and an lgkmcnt wait before the
first use of every LDS load (at most 15 in flight).

Usage: python3 gen_w64_loop.py [out] [--kpre N] [--vpre N] [--per1 N] [--check-at N] [--[no-]check-spread]
(default out: kd_fa_w64_loop.inc beside it).  The schedule knobs are
tuning switches for variant builds; the committed loop uses the defaults,
and the environment is never read.
"""
import argparse
import copy
import os
import re

# ---------------------------------------------------------------- registers
# VGPRs v24..v247 belong to the loop; the compiler keeps v0..v23 and
# v248..v255 for the operands and its own values.
S_BASE = (24, 88)      # S[parity]: [qb][kb] -> +32*qb + 16*kb, 16 floats
P_BASE = (152, 184)    # P[parity]: [qb][kst] -> +16*qb + 4*kst, 4 words
T_BASE = 216           # 4 fma results
E_BASE = 220           # 8 exp results
M = (228, 229)         # running max per query block (log2 units)
LH = (230, 231)        # running half-row weight sum
# per query block: the tile's half-row weight sum (keys 0-31 first, then all
# 64) and two partial sums of 16-key steps
PS = ((232, 233, 234), (235, 236, 237))
X, Y = 238, 239
W_BASE = 240           # slow-path temporaries (240..247)
V_LAST = 247
# AGPRs
A_O = 0                # O[qb][dblk] -> +64*qb + 16*dblk, 16 floats
A_Q = 128              # Q[qb][ks] -> +32*qb + 4*ks
# LDS operand prefetch distances: K fragments KPRE k-steps ahead, V^T
# fragments VPRE fragments ahead (ring slots: KPRE + 1 and VPRE + 2); set by
# configure() from the command line
KPRE = VPRE = A_VF = A_LAST = None
A_KF = 192             # K fragments: (KPRE + 1) slots x 2 key blocks x 4
# SGPRs s84..s95
S_K = 84               # s[84:87] K buffer resource (moves one tile per DMA)
S_V = 88               # s[88:91] V buffer resource
S_T = 92               # step counter
S_TMP = 93
S_VCC = 94             # s[94:95]: the row check's lane mask
S_FIRST, S_LAST = 84, 95

# LDS layout (bytes from the workgroup's array)
KBUF = (0, 16384)
VBUF = (32768, 49152)
Q_OFF = 65536

# Phase 1 schedule: VALU instructions after each MFMA, and the MFMA before
# which the row check starts (the rest of S(t+1) is computed meanwhile)
PER1 = CHECK_AT = None
# Row check spread over the last MFMAs of phase 1: its dependent chain (moves,
# lane swap, add, compare) one group per MFMA from MFMA CHECK_AT on, the
# branch after the last MFMA
CHECK_SPREAD = False

# Row-sum cap of the lazy running max, as an F32 bit pattern: the weights are
# rounded to the operand type for PV, so the cap stays inside its range
SUM_CAP = {"bf16": "0x5f800000",   # 2^64
           "f16": "0x47000000"}    # 2^15 (F16's largest finite value is 65504)


def configure(kpre=2, vpre=2, per1=4, check_at=29, check_spread=True):
    global KPRE, VPRE, A_VF, A_LAST, PER1, CHECK_AT, CHECK_SPREAD
    KPRE, VPRE, PER1, CHECK_AT, CHECK_SPREAD = kpre, vpre, per1, check_at, check_spread
    A_VF = A_KF + 8 * (KPRE + 1)   # V^T fragments: (VPRE + 2) slots x 4
    A_LAST = A_VF + 4 * (VPRE + 2) - 1
    assert A_LAST <= 255


configure()

MFMA_WS = 20           # MFMA result -> VALU / LDS / accvgpr access
VALU_MFMA_WS = 4       # VALU or accvgpr write -> MFMA operand read
TRANS_WS = 2           # v_exp result -> reader
DOT_WS = 3             # v_dot2 result -> reader other than a dot2 accumulating on it
DOT_ACC_WS = 2         # v_dot2 result -> the next dot2 of its chain
PERM_WS = 2            # VALU write -> v_permlane32_swap read
M0_WS = 1              # m0 write -> LDS DMA


def vr(i):
    return f"v{i}"


def vrng(b, n):
    return f"v[{b}:{b + n - 1}]"


def arng(b, n):
    return f"a[{b}:{b + n - 1}]"


def vset(b, n):
    return {f"v{i}" for i in range(b, b + n)}


def aset(b, n):
    return {f"a{i}" for i in range(b, b + n)}


class Ins:
    """One instruction: text, kind, registers read and written."""

    def __init__(self, text, kind, rd=(), wr=(), m0w=False, m0r=False):
        self.text, self.kind = text, kind
        self.rd, self.wr = set(rd), set(wr)
        self.m0w, self.m0r = m0w, m0r


def valu(text, rd, wr):
    return Ins(text, "valu", rd, wr)


class Tracker:
    """Inserts s_nop / s_waitcnt lgkmcnt in straight-line code."""

    def __init__(self):
        self.out = []
        self.pos = 0
        self.mfma_w = {}
        self.valu_w = {}
        self.trans_w = {}
        self.dot_w = {}
        self.m0_w = -100
        self.lds = []       # pending LDS ops: (regs written, regs read)

    def _nop(self, n):
        while n > 0:
            k = min(n, 8)
            self.out.append(f"s_nop {k - 1}")
            self.pos += k
            n -= k

    def _wait_lgkm(self, keep):
        self.out.append(f"s_waitcnt lgkmcnt({keep})")
        self.pos += 1
        self.lds = self.lds[len(self.lds) - keep:] if keep else []

    def label(self, name):
        self.out.append(f"{name}:")

    def raw(self, text, ws=1):
        self.out.append(text)
        self.pos += ws

    def emit(self, i):
        touched = i.rd | i.wr
        # LDS results: wait for the last pending load this instruction touches
        last = -1
        for k, (w, r) in enumerate(self.lds):
            if (w & touched) or (r & i.wr):
                last = k
        if last >= 0:
            self._wait_lgkm(len(self.lds) - last - 1)
        if i.kind in ("lds_rd", "lds_wr") and len(self.lds) >= 15:
            self._wait_lgkm(14)
        need = 0
        if i.kind != "mfma":
            for r in touched:
                if r in self.mfma_w:
                    need = max(need, MFMA_WS - (self.pos - self.mfma_w[r] - 1))
        else:
            for r in i.rd:
                if r in self.valu_w:
                    need = max(need, VALU_MFMA_WS - (self.pos - self.valu_w[r] - 1))
        for r in i.rd:
            if r in self.trans_w:
                need = max(need, TRANS_WS - (self.pos - self.trans_w[r] - 1))
        for r in i.rd:
            if r in self.dot_w:
                ws = DOT_ACC_WS if (i.kind == "dot" and r in i.wr) else DOT_WS
                need = max(need, ws - (self.pos - self.dot_w[r] - 1))
        if i.kind == "perm":
            for r in i.rd:
                if r in self.valu_w:
                    need = max(need, PERM_WS - (self.pos - self.valu_w[r] - 1))
        if i.m0r:
            need = max(need, M0_WS - (self.pos - self.m0_w - 1))
        if need > 0:
            self._nop(need)
        self.out.append(i.text)
        p = self.pos
        self.pos += 1
        if i.m0w:
            self.m0_w = p
        for r in i.wr:
            self.mfma_w.pop(r, None)
            self.valu_w.pop(r, None)
            self.trans_w.pop(r, None)
            self.dot_w.pop(r, None)
        if i.kind == "mfma":
            for r in i.wr:
                self.mfma_w[r] = p
        elif i.kind in ("valu", "trans", "perm", "accw", "dot"):
            for r in i.wr:
                self.valu_w[r] = p
            if i.kind == "trans":
                for r in i.wr:
                    self.trans_w[r] = p
            if i.kind == "dot":
                for r in i.wr:
                    self.dot_w[r] = p
        if i.kind == "lds_rd":
            self.lds.append((set(i.wr), set()))
        elif i.kind == "lds_wr":
            self.lds.append((set(), set(i.rd)))

    def settle(self):
        """Forget hazards older than any rule's window (after barriers)."""
        horizon = self.pos - 64
        for d in (self.mfma_w, self.valu_w, self.trans_w, self.dot_w):
            for r in [r for r, p in d.items() if p < horizon]:
                del d[r]


class Gen:
    def __init__(self, T):
        self.T = T
        self.mfma = f"v_mfma_f32_32x32x16_{T}"
        self.cvt = {"bf16": "v_cvt_pk_bf16_f32", "f16": "v_cvt_pk_f16_f32"}[T]
        self.slow = []      # out-of-line blocks (lists of lines)

    # ---------------------------------------------------------- streams
    def qk_stream(self, kbuf, sp):
        """S[sp] = K(kbuf) Q^T: (pre-reads, [(reads before, mfma)])."""
        reads = {}
        for ks in range(8):
            slot = ks % (KPRE + 1)
            reads[ks] = [Ins(f"ds_read_b128 {arng(A_KF + 8 * slot + 4 * kb, 4)}, %[krd{ks}] offset:{kbuf + kb * 8192}",
                             "lds_rd", (), aset(A_KF + 8 * slot + 4 * kb, 4)) for kb in range(2)]
        pre = sum((reads[ks] for ks in range(KPRE)), [])
        seq = []
        for ks in range(8):
            slot = ks % (KPRE + 1)
            n = 0
            for kb in range(2):
                for qb in range(2):
                    d = S_BASE[sp] + 32 * qb + 16 * kb
                    a = A_KF + 8 * slot + 4 * kb
                    b = A_Q + 32 * qb + 4 * ks
                    c = "0" if ks == 0 else vrng(d, 16)
                    rd = aset(a, 4) | aset(b, 4) | (set() if ks == 0 else vset(d, 16))
                    before = reads[ks + KPRE] if (n == 1 and ks + KPRE < 8) else []
                    seq.append((before, Ins(f"{self.mfma} {vrng(d, 16)}, {arng(a, 4)}, {arng(b, 4)}, {c}",
                                            "mfma", rd, vset(d, 16))))
                    n += 1
        return pre, seq

    def pv_stream(self, vbuf, pp):
        """O += V(vbuf)^T P[pp]^T: (pre-reads, [(reads before, mfma)])."""
        def frag_reads(f):
            kst, dblk = divmod(f, 4)
            s = A_VF + 4 * (f % (VPRE + 2))
            off = vbuf + 4096 * kst
            return [Ins(f"ds_read_b64_tr_b16 {arng(s, 2)}, %[vrd{dblk}] offset:{off}", "lds_rd", (), aset(s, 2)),
                    Ins(f"ds_read_b64_tr_b16 {arng(s + 2, 2)}, %[vrd{dblk}] offset:{off + 1024}", "lds_rd", (),
                        aset(s + 2, 2))]
        pre = sum((frag_reads(f) for f in range(VPRE)), [])
        seq = []
        for f in range(16):
            kst, dblk = divmod(f, 4)
            s = A_VF + 4 * (f % (VPRE + 2))
            for qb in range(2):
                o = A_O + 64 * qb + 16 * dblk
                p = P_BASE[pp] + 16 * qb + 4 * kst
                before = frag_reads(f + VPRE) if (qb == 1 and f + VPRE < 16) else []
                seq.append((before, Ins(f"{self.mfma} {arng(o, 16)}, {arng(s, 4)}, {vrng(p, 4)}, {arng(o, 16)}",
                                        "mfma", aset(o, 16) | aset(s, 4) | vset(p, 4), aset(o, 16))))
        return pre, seq

    def softmax_half(self, sp, pp, half, qbs, finish):
        """VALU stream: weights of keys 32*half .. +31 of S[sp] for the query
        blocks qbs (pairs of blocks interleaved), rounded into P[pp]; each
        16-key step's row sum adds its 8 F32 weights in order (one add chain
        per step).  finish: half 0 leaves s0 + s1 in PS[qb][0]; half 1 leaves
        (s0 + s1) + (s2 + s3) there."""
        pairs = [(qb, k) for k in range(8) for qb in qbs]
        n = len(pairs)
        out = []
        for i in range(n + 2):
            if i < n:
                qb, k = pairs[i]
                sb = S_BASE[sp] + 32 * qb + 16 * half
                t = T_BASE + 2 * (i % 2)
                for h in range(2):
                    out.append(valu(f"v_fma_f32 {vr(t + h)}, {vr(sb + 2 * k + h)}, |%[c2]|, -{vr(M[qb])}",
                                    {vr(sb + 2 * k + h), vr(M[qb])}, {vr(t + h)}))
            if 1 <= i <= n:
                t = T_BASE + 2 * ((i - 1) % 2)
                e = E_BASE + 2 * ((i - 1) % 4)
                for h in range(2):
                    out.append(Ins(f"v_exp_f32 {vr(e + h)}, {vr(t + h)}", "trans", {vr(t + h)}, {vr(e + h)}))
            if i >= 2:
                qb, k = pairs[i - 2]
                e = E_BASE + 2 * ((i - 2) % 4)
                kst, j = 2 * half + k // 4, k % 4
                w = P_BASE[pp] + 16 * qb + 4 * kst + j
                acc = PS[qb][1 + (kst & 1)]
                out.append(valu(f"{self.cvt} {vr(w)}, {vr(e)}, {vr(e + 1)}", {vr(e), vr(e + 1)}, {vr(w)}))
                if j == 0:
                    out.append(valu(f"v_add_f32 {vr(acc)}, {vr(e)}, {vr(e + 1)}", {vr(e), vr(e + 1)}, {vr(acc)}))
                else:
                    for h in range(2):
                        out.append(valu(f"v_add_f32 {vr(acc)}, {vr(acc)}, {vr(e + h)}", {vr(acc), vr(e + h)}, {vr(acc)}))
        for qb in qbs:
            h01, a, b = PS[qb]
            if half == 0:
                out.append(valu(f"v_add_f32 {vr(h01)}, {vr(a)}, {vr(b)}", {vr(a), vr(b)}, {vr(h01)}))
            else:
                out.append(valu(f"v_add_f32 {vr(a)}, {vr(a)}, {vr(b)}", {vr(a), vr(b)}, {vr(a)}))
                out.append(valu(f"v_add_f32 {vr(h01)}, {vr(h01)}, {vr(a)}", {vr(a), vr(h01)}, {vr(h01)}))
        return out

    def dma(self, which, buf, j):
        base = S_K if which == "k" else S_V
        return [Ins(f"s_add_u32 m0, %[dmab], {buf + 4096 * j}", "salu", m0w=True),
                Ins(f"buffer_load_dwordx4 %[{which}dma{j}], s[{base}:{base + 3}], 0 offen lds", "vmem", m0r=True)]

    def advance(self, which):
        base = S_K if which == "k" else S_V
        tile = "%[ktile]" if which == "k" else "%[vtile]"
        return [Ins(f"s_add_u32 s{base}, s{base}, {tile}", "salu"),
                Ins(f"s_addc_u32 s{base + 1}, s{base + 1}, 0", "salu"),
                Ins(f"s_sub_u32 s{base + 2}, s{base + 2}, {tile}", "salu"),
                Ins(f"s_cselect_b32 s{base + 2}, 0, s{base + 2}", "salu")]

    # ------------------------------------------------------------ pieces
    def merge(self, tr, seq, valus, extra=(), per=3, tail=None, tail_at=None, spread=(), end=None):
        """MFMAs in order, reads ahead of them, `per` VALU after each,
        `extra` (SALU/VMEM groups) one group after each of the first MFMAs;
        `tail` (emitting code) after MFMA tail_at - 1 and all of `valus`;
        then the groups of `spread` one after each later MFMA, and `end`
        (emitting code) after the last MFMA."""
        vi = 0
        extra = list(extra)
        spread = list(spread)
        tail_at = len(seq) if tail_at is None else tail_at

        def finish():
            nonlocal vi
            for grp in extra:
                for x in grp:
                    tr.emit(x)
            extra.clear()
            while vi < len(valus):
                tr.emit(valus[vi])
                vi += 1
            if tail:
                tail(tr)

        for n, (before, m) in enumerate(seq):
            if n == tail_at:
                finish()
            for r in before:
                tr.emit(r)
            tr.emit(m)
            if n >= 1 and extra:
                for x in extra.pop(0):
                    tr.emit(x)
            if n < tail_at:
                for _ in range(per):
                    if vi < len(valus):
                        tr.emit(valus[vi])
                        vi += 1
            elif spread:
                for x in spread.pop(0):
                    tr.emit(x)
        if tail_at >= len(seq):
            finish()
        for grp in spread:
            for x in grp:
                tr.emit(x)
        if end:
            end(tr)

    def check_groups(self, p, tag):
        """Row-sum check of both query blocks: one v_permlane32_swap of the
        two blocks' half sums gives block 0's row sums in lanes 0-31 and
        block 1's in lanes 32-63; the slow paths are out of line.  Returns
        the groups of the dependent chain and the code of the branch."""
        s0, s1 = PS[0][0], PS[1][0]
        groups = [[valu(f"v_mov_b32 {vr(X)}, {vr(s0)}", {vr(s0)}, {vr(X)}),
                   valu(f"v_mov_b32 {vr(Y)}, {vr(s1)}", {vr(s1)}, {vr(Y)})],
                  [Ins(f"v_permlane32_swap_b32 {vr(X)}, {vr(Y)}", "perm", {vr(X), vr(Y)}, {vr(X), vr(Y)})],
                  [valu(f"v_add_f32 {vr(X)}, {vr(X)}, {vr(Y)}", {vr(X), vr(Y)}, {vr(X)}),
                   valu(f"v_cmp_nge_f32 vcc, {SUM_CAP[self.T]}, {vr(X)}", {vr(X)}, ())]]
        return groups, lambda tr: self.check_branch(tr, p, tag)

    def check(self, tr, p, tag):
        groups, branch = self.check_groups(p, tag)
        for grp in groups:
            for x in grp:
                tr.emit(x)
        branch(tr)

    def check_branch(self, tr, p, tag):
        slow, back = f".Lw64_slow_{tag}_%=", f".Lw64_back_{tag}_%="
        tr.emit(Ins(f"s_cbranch_vccnz {slow}", "branch"))
        tr.label(back)
        for qb in range(2):
            tr.emit(valu(f"v_add_f32 {vr(LH[qb])}, {vr(LH[qb])}, {vr(PS[qb][0])}", {vr(LH[qb]), vr(PS[qb][0])},
                         {vr(LH[qb])}))
        blk = [f"{slow}:", f"s_mov_b64 s[{S_VCC}:{S_VCC + 1}], vcc"]
        for qb in range(2):
            skip = f".Lw64_skip_{tag}{qb}_%="
            blk += [f"s_cmp_lg_u32 s{S_VCC + qb}, 0", f"s_cbranch_scc0 {skip}"]
            blk += self.slow_block(p, qb, f"{tag}{qb}")
            blk += [f"{skip}:"]
        blk += ["s_nop 7", f"s_branch {back}"]
        self.slow.append(blk)

    @staticmethod
    def row_max(e, p, qb, w):
        """X = the exact row max of S[p][qb] over the lane pair, times |c2|
        (w: three temporaries)."""
        sb = S_BASE[p] + 32 * qb
        s = [vr(sb + i) for i in range(32)]
        e(valu(f"v_max3_f32 {vr(w[0])}, {s[0]}, {s[1]}, {s[2]}", set(s[0:3]), {vr(w[0])}))
        e(valu(f"v_max3_f32 {vr(w[1])}, {s[3]}, {s[4]}, {s[5]}", set(s[3:6]), {vr(w[1])}))
        for i in range(6, 30, 4):
            e(valu(f"v_max3_f32 {vr(w[0])}, {vr(w[0])}, {s[i]}, {s[i + 1]}", {vr(w[0]), s[i], s[i + 1]}, {vr(w[0])}))
            e(valu(f"v_max3_f32 {vr(w[1])}, {vr(w[1])}, {s[i + 2]}, {s[i + 3]}", {vr(w[1]), s[i + 2], s[i + 3]},
                   {vr(w[1])}))
        e(valu(f"v_max_f32 {vr(w[2])}, {s[30]}, {s[31]}", {s[30], s[31]}, {vr(w[2])}))
        e(valu(f"v_max3_f32 {vr(w[0])}, {vr(w[0])}, {vr(w[1])}, {vr(w[2])}", {vr(w[0]), vr(w[1]), vr(w[2])},
               {vr(w[0])}))
        # max over the lane pair, times |c2|
        e(valu(f"v_mov_b32 {vr(X)}, {vr(w[0])}", {vr(w[0])}, {vr(X)}))
        e(valu(f"v_mov_b32 {vr(Y)}, {vr(w[0])}", {vr(w[0])}, {vr(Y)}))
        e(Ins(f"v_permlane32_swap_b32 {vr(X)}, {vr(Y)}", "perm", {vr(X), vr(Y)}, {vr(X), vr(Y)}))
        e(valu(f"v_max_f32 {vr(X)}, {vr(X)}, {vr(Y)}", {vr(X), vr(Y)}, {vr(X)}))
        e(valu(f"v_mul_f32 {vr(X)}, |%[c2]|, {vr(X)}", {vr(X)}, {vr(X)}))

    def slow_block(self, p, qb, tag):
        """Exact row max of S[p][qb]; the rows whose own weight sum failed
        the check move to it, with O and the sums rescaled; all 32 weights
        again (move_max and the slow path of soft_pv in kd_fa_kernel.hip)."""
        tr = Tracker()
        sb = S_BASE[p] + 32 * qb
        w = [W_BASE + i for i in range(7)]
        s = [vr(sb + i) for i in range(32)]
        e = tr.emit
        e(valu(f"v_max3_f32 {vr(w[0])}, {s[0]}, {s[1]}, {s[2]}", set(s[0:3]), {vr(w[0])}))
        e(valu(f"v_max3_f32 {vr(w[1])}, {s[3]}, {s[4]}, {s[5]}", set(s[3:6]), {vr(w[1])}))
        for i in range(6, 30, 4):
            e(valu(f"v_max3_f32 {vr(w[0])}, {vr(w[0])}, {s[i]}, {s[i + 1]}", {vr(w[0]), s[i], s[i + 1]}, {vr(w[0])}))
            e(valu(f"v_max3_f32 {vr(w[1])}, {vr(w[1])}, {s[i + 2]}, {s[i + 3]}", {vr(w[1]), s[i + 2], s[i + 3]},
                   {vr(w[1])}))
        e(valu(f"v_max_f32 {vr(w[2])}, {s[30]}, {s[31]}", {s[30], s[31]}, {vr(w[2])}))
        e(valu(f"v_max3_f32 {vr(w[0])}, {vr(w[0])}, {vr(w[1])}, {vr(w[2])}", {vr(w[0]), vr(w[1]), vr(w[2])},
               {vr(w[0])}))
        # max over the lane pair, times |c2|
        e(valu(f"v_mov_b32 {vr(X)}, {vr(w[0])}", {vr(w[0])}, {vr(X)}))
        e(valu(f"v_mov_b32 {vr(Y)}, {vr(w[0])}", {vr(w[0])}, {vr(Y)}))
        e(Ins(f"v_permlane32_swap_b32 {vr(X)}, {vr(Y)}", "perm", {vr(X), vr(Y)}, {vr(X), vr(Y)}))
        e(valu(f"v_max_f32 {vr(X)}, {vr(X)}, {vr(Y)}", {vr(X), vr(Y)}, {vr(X)}))
        e(valu(f"v_mul_f32 {vr(X)}, |%[c2]|, {vr(X)}", {vr(X)}, {vr(X)}))
        # a row's running max moves when the row's own weight sum failed
        # the check: bit r of the block's check mask (row r sits in lanes r
        # and r + 32), as the lane mask of both halves.  This block runs
        # only when that mask is not empty.
        e(Ins(f"s_mov_b32 vcc_lo, s{S_VCC + qb}", "salu"))
        e(Ins(f"s_mov_b32 vcc_hi, s{S_VCC + qb}", "salu"))
        e(Ins("s_nop 1", "salu"))
        e(valu(f"v_max_f32 {vr(Y)}, {vr(M[qb])}, {vr(X)}", {vr(M[qb]), vr(X)}, {vr(Y)}))
        e(valu(f"v_cndmask_b32 {vr(Y)}, {vr(M[qb])}, {vr(Y)}, vcc", {vr(M[qb]), vr(Y)}, {vr(Y)}))   # m_new
        e(valu(f"v_sub_f32 {vr(w[2])}, {vr(M[qb])}, {vr(Y)}", {vr(M[qb]), vr(Y)}, {vr(w[2])}))
        e(Ins(f"v_exp_f32 {vr(w[2])}, {vr(w[2])}", "trans", {vr(w[2])}, {vr(w[2])}))
        e(valu(f"v_cmp_neq_f32 vcc, {vr(Y)}, {vr(M[qb])}", {vr(Y), vr(M[qb])}, ()))
        e(valu(f"v_cndmask_b32 {vr(w[2])}, 1.0, {vr(w[2])}, vcc", {vr(w[2])}, {vr(w[2])}))          # alpha
        e(valu(f"v_mov_b32 {vr(M[qb])}, {vr(Y)}", {vr(Y)}, {vr(M[qb])}))
        e(valu(f"v_mul_f32 {vr(LH[qb])}, {vr(LH[qb])}, {vr(w[2])}", {vr(LH[qb]), vr(w[2])}, {vr(LH[qb])}))
        tmp = w[3:7]
        for c in range(0, 64, 4):
            for i in range(4):
                a = f"a{A_O + 64 * qb + c + i}"
                e(Ins(f"v_accvgpr_read_b32 {vr(tmp[i])}, {a}", "valu", {a}, {vr(tmp[i])}))
            for i in range(4):
                e(valu(f"v_mul_f32 {vr(tmp[i])}, {vr(tmp[i])}, {vr(w[2])}", {vr(tmp[i]), vr(w[2])}, {vr(tmp[i])}))
            for i in range(4):
                a = f"a{A_O + 64 * qb + c + i}"
                e(Ins(f"v_accvgpr_write_b32 {a}, {vr(tmp[i])}", "accw", {vr(tmp[i])}, {a}))
        for x in self.softmax_half(p, p, 0, (qb,), True) + self.softmax_half(p, p, 1, (qb,), True):
            e(x)
        return tr.out

    # -------------------------------------------------------------- step
    def mask_tail(self, tr, q, toff, tag):
        """In the step whose S(t+1) is the partial last tile (t = S_T + toff
        equals the operand mstep), scores of keys >= Lk in S[q] -> -inf.
        thr (per lane) = valid keys of the tile - 8 * (lane / 32): register
        i of key block kb holds key 32 kb + 16 ((i / 8) % 2) + 8 (lane / 32)
        + i % 8 of the tile.  The block's wait states are counted on a copy
        of the tracker; the tracker itself goes on as on the path that skips
        the block (the taken path only adds distance, and its writes are
        VALU results that only VALU instructions read)."""
        skip = f".Lw64_nomask_{tag}_%="
        if toff:
            tr.raw(f"s_add_u32 s{S_TMP}, s{S_T}, {toff}")
            tr.raw(f"s_cmp_eq_u32 s{S_TMP}, %[mstep]")
        else:
            tr.raw(f"s_cmp_eq_u32 s{S_T}, %[mstep]")
        tr.raw(f"s_cbranch_scc0 {skip}")
        tb = copy.deepcopy(tr)
        n0 = len(tb.out)
        ninf = vr(W_BASE)      # a slow-path temporary, free here
        tb.emit(valu(f"v_mov_b32 {ninf}, 0xff800000", (), {ninf}))
        for kb in range(2):
            for i in range(16):
                c = 32 * kb + 16 * ((i >> 3) & 1) + (i & 7)
                tb.emit(valu(f"v_cmp_lt_i32 vcc, {c}, %[thr]", (), ()))
                for qb in range(2):
                    r = vr(S_BASE[q] + 32 * qb + 16 * kb + i)
                    tb.emit(valu(f"v_cndmask_b32 {r}, {ninf}, {r}, vcc", {r, ninf}, {r}))
        tr.out.extend(tb.out[n0:])
        tr.label(skip)

    def step(self, tr, p, final, tag, toff=0, unit=False):
        """Step t = S_T + toff with parity p: S(t) in S[p], K(t+1) in
        KBUF[1-p], V(t) in VBUF[p]; P[p] holds the weights of keys 0-31 of
        tile t.  unit: a step of the persistent kernel's unit block (the
        next unit's Q pieces in steps 0-4; the last step fetches the next
        unit's K(0) and K(1))."""
        q = 1 - p
        vpre, vseq = self.pv_stream(VBUF[p], p)

        def tail(tr):
            for r in vpre:
                tr.emit(r)
            self.check(tr, p, tag)
            if unit and final:
                self.piece_block(tr, p, toff, tag)

        if not final:
            pre, seq = self.qk_stream(KBUF[q], q)
            for r in pre:
                tr.emit(r)
            dmas = [self.dma("v", VBUF[q], j) for j in range(4)] + [self.advance("v")] + \
                   [self.dma("k", KBUF[p], j) for j in range(4)] + [self.advance("k")]
            if CHECK_SPREAD:
                groups, branch = self.check_groups(p, tag)

                def head(tr):
                    for r in vpre:
                        tr.emit(r)
                    for x in groups[0]:
                        tr.emit(x)

                self.merge(tr, seq, self.softmax_half(p, p, 1, (0, 1), True), dmas, PER1, head, CHECK_AT,
                           groups[1:], branch)
            else:
                self.merge(tr, seq, self.softmax_half(p, p, 1, (0, 1), True), dmas, PER1, tail, CHECK_AT)
        else:
            if unit:
                self.next_k(tr)
            for x in self.softmax_half(p, p, 1, (0, 1), True):
                tr.emit(x)
            tail(tr)
        if not final:
            self.mask_tail(tr, q, toff, tag)
            if unit:
                self.piece_block(tr, p, toff, tag)
            self.merge(tr, vseq, self.softmax_half(q, q, 0, (0, 1), True))
            if unit:
                self.step_wait(tr, toff, tag)
            else:
                tr.raw("s_waitcnt vmcnt(0)")
            tr.raw("s_barrier")
            tr.settle()
        else:
            self.merge(tr, vseq, [])

    def first_tiles(self, e, dma):
        """The K and V resources from the operands, moved past K(0), V(0)
        and K(1) -- with dma, also the DMAs of those tiles (a DMA past the
        last tile reads zeros: the resource's record count is clamped at
        0)."""
        for j, w in enumerate(("kw0", "kw1", "kw2", "kw3")):
            e(Ins(f"s_mov_b32 s{S_K + j}, %[{w}]", "salu"))
        for j, w in enumerate(("vw0", "vw1", "vw2", "vw3")):
            e(Ins(f"s_mov_b32 s{S_V + j}, %[{w}]", "salu"))
        for which, buf in (("k", KBUF[0]), ("v", VBUF[0]), ("k", KBUF[1])):
            if dma:
                for j in range(4):
                    for x in self.dma(which, buf, j):
                        e(x)
            for x in self.advance(which):
                e(x)

    def build_pre(self):
        """The block fa_fwd_w64 runs before its Q loads: the DMAs of K(0),
        V(0) and K(1), so that their round trip overlaps the Q load's (the
        kernel's wait for its Q loads, which come later in the same in-order
        counter, covers them)."""
        tr = Tracker()
        self.first_tiles(tr.emit, dma=True)
        return tr.out

    def build(self):
        tr = Tracker()
        e = tr.emit
        for qb in range(2):
            e(valu(f"v_mov_b32 {vr(M[qb])}, 0xff800000", (), {vr(M[qb])}))
            e(valu(f"v_mov_b32 {vr(LH[qb])}, 0", (), {vr(LH[qb])}))
        for i in range(128):
            e(Ins(f"v_accvgpr_write_b32 a{A_O + i}, 0", "accw", (), {f"a{A_O + i}"}))
        for i in range(16):
            e(Ins(f"ds_read_b128 {arng(A_Q + 4 * i, 4)}, %[qrd] offset:{1024 * i}", "lds_rd", (), aset(A_Q + 4 * i, 4)))
        # K(0), V(0), K(1) were issued by build_pre's block, ahead of the
        # kernel's Q loads; here the resources only move past them
        self.first_tiles(e, dma=False)
        tr.raw("s_waitcnt vmcnt(0) lgkmcnt(0)")
        tr.lds = []
        tr.raw("s_barrier")
        # S(0), then every wave is done with K(0) before K(2) lands there
        pre, seq = self.qk_stream(KBUF[0], 0)
        for r in pre:
            e(r)
        self.merge(tr, seq, [])
        tr.raw("s_barrier")
        # step 0's exact row max: against the running max of -inf every
        # weight of S(0) would be +inf, fail step 0's check and be redone on
        # the slow path against this max (O and the sums, still 0, need no
        # rescale); max(-inf, X) as the slow path's move gives it
        for qb in range(2):
            self.row_max(e, 0, qb, [W_BASE + i for i in range(3)])
            e(valu(f"v_max_f32 {vr(M[qb])}, {vr(M[qb])}, {vr(X)}", {vr(M[qb]), vr(X)}, {vr(M[qb])}))
        for x in self.softmax_half(0, 0, 0, (0, 1), True):
            e(x)
        # steps: pairs while t + 2 < n, then one or two more
        tr.raw(f"s_mov_b32 s{S_T}, 0")
        tr.label(".Lw64_loop_%=")
        tr.raw(f"s_add_u32 s{S_TMP}, s{S_T}, 2")
        tr.raw(f"s_cmp_lt_u32 s{S_TMP}, %[n]")
        tr.raw(".Lw64_tail_%=".join(["s_cbranch_scc0 ", ""]))
        self.step(tr, 0, False, "a", 0)
        self.step(tr, 1, False, "b", 1)
        tr.raw(f"s_add_u32 s{S_T}, s{S_T}, 2")
        tr.raw("s_branch .Lw64_loop_%=")
        tr.label(".Lw64_tail_%=")
        tr.raw(f"s_add_u32 s{S_TMP}, s{S_T}, 1")
        tr.raw(f"s_cmp_lt_u32 s{S_TMP}, %[n]")
        tr.raw("s_cbranch_scc0 .Lw64_last0_%=")
        self.step(tr, 0, False, "c", 0)
        self.step(tr, 1, True, "d")
        tr.raw("s_branch .Lw64_done_%=")
        tr.label(".Lw64_last0_%=")
        self.step(tr, 0, True, "e")
        tr.label(".Lw64_done_%=")
        # O / l -> the rows, staged over the K/V tiles once every wave is
        # done with them
        self.epilogue(tr, next_v=False)
        tr.raw("s_branch .Lw64_end_%=")
        lines = tr.out
        for blk in self.slow:
            lines += blk
        lines.append(".Lw64_end_%=:")
        return lines


# ------------------------------------------------- persistent unit block
# fa_fwd_xlong64 (kd_fa_kernel.hip) runs the loop above once per unit of 256
# query rows of one (b, h) and walks several units per workgroup; its block
# adds, per unit, the next unit's Q (F32 rows brought in by DMA during the
# first steps and rounded into the Q fragment area; Q stored in the operand
# type DMA'd into it as it is), the next unit's first
# K/V tiles (issued by the last step and after it) and the O epilogue
# (normalised rows staged in LDS, stored as whole 128-byte lines through a
# buffer resource whose record count ends at the last valid row).
XL_QF = 65536          # Q fragments: per wave 16 KiB (the loop's Q_OFF layout)
XL_RAW = 131072        # per wave 8 KiB: raw Q pieces in the loop, O staging after it
XL_RAW_W = 8192
XL_PIECES = 4          # 128-byte pieces of an F32 row, one per step in steps 0-3
XL_PIECE_DMAS = 8      # DMA instructions per piece and wave
XL_KV_DMAS = 8         # K/V DMA instructions per step and wave (the last step: K(0), K(1) of the next unit)
XL_Q16_DMAS = 4        # Q in the operand type: fragment DMAs per step and wave (steps 0-3)
XL_PITCH = 144         # O staging: bytes per row (128 + 16: no bank conflicts)
S_NQ = 80              # s[80:83] the next unit's Q buffer resource
S_T2, S_T3 = 96, 97    # temporaries of the unit block
XL_S_FIRST, XL_S_LAST = 80, 97
# epilogue VGPRs (the loop's are free by then, except the half-row sums LH)
EP_INV = (216, 217)
EP_T = list(range(218, 228))
EP_LANE = 228
EP_STW, EP_STW16, EP_STR, EP_OOFF = 229, 234, 232, 233
EP_OROW = list(range(240, 248))
XL_STORES = {"f32": 32, "b16": 16}   # O stores per wave and unit


def _xl_unit_methods():
    """Methods of Gen for the unit block (kept apart from the loop's)."""

    def next_k(self, tr):
        """The last step of a unit: the next unit's K(0) and K(1) into the K
        buffers (no wave reads them any more: the previous step's barrier has
        passed); record count 0 when there is no next unit (zeros)."""
        for j, w in enumerate(("nkw0", "nkw1", "nkw2", "rw3")):
            tr.emit(Ins(f"s_mov_b32 s{S_K + j}, %[{w}]", "salu"))
        for j in range(4):
            for x in self.dma("k", KBUF[0], j):
                tr.emit(x)
        for x in self.advance("k"):
            tr.emit(x)
        for j in range(4):
            for x in self.dma("k", KBUF[1], j):
                tr.emit(x)

    def piece_index(self, tr, toff):
        """s[S_T2] = the step index t = S_T + toff."""
        if toff:
            tr.raw(f"s_add_u32 s{S_T2}, s{S_T}, {toff}")
        else:
            tr.raw(f"s_mov_b32 s{S_T2}, s{S_T}")

    def step_wait(self, tr, toff, tag):
        """The end of a non-final step t: its K/V DMAs done.  In steps 0-3
        the piece DMAs issued after them (XL_PIECE_DMAS) stay in flight:
        the conversion a step later waits for them, so that their memory
        latency overlaps a whole step."""
        # (steps past the pieces fall through: one compare, no taken branch)
        wp, wd = f".Lxl_wp_{tag}_%=", f".Lxl_wd_{tag}_%="
        tr.raw(f"s_cmp_le_u32 s{S_T}, {XL_PIECES - 1 - toff}")
        tr.raw(f"s_cbranch_scc1 {wp}")
        tr.raw("s_waitcnt vmcnt(0)")
        tr.label(wd)
        self.slow.append([f"{wp}:", f"s_waitcnt vmcnt({XL_Q16_DMAS if self.q16 else XL_PIECE_DMAS})",
                          f"s_branch {wd}"])

    def piece_block(self, tr, p, toff, tag):
        """The next unit's Q work of step t = S_T + toff, out of line: steps
        0-4 branch to it, the others fall through on one compare.  The body
        (piece_block_f32 / piece_block_q16) uses the dead score registers
        S[p] and the free SGPRs and goes on a tracker of its own; the main
        tracker goes on as on the path that skips it: the body's LDS
        operations left pending are fragment writes, older than any LDS
        operation a later wait is for."""
        R = S_BASE[p]
        skip = f".Lxl_nopiece_{tag}_%="
        body = f".Lxl_piece_{tag}_%="
        tr.raw(f"s_cmp_le_u32 s{S_T}, {XL_PIECES - toff}")
        tr.raw(f"s_cbranch_scc1 {body}")
        tr.label(skip)
        tb = Tracker()
        tb.label(body)
        if self.q16:
            self.piece_block_q16(tb, R, toff, tag)
        else:
            self.piece_block_f32(tb, R, toff, tag)
        tb.raw(f"s_branch {skip}")
        self.slow.append(tb.out)

    def piece_block_f32(self, tr, R, toff, tag):
        """F32 Q, step t <= 4: piece t - 1 of the next unit's rows (t >= 1)
        from the raw area, rounded to the operand type (with load_q_frags'
        sign for scale < 0) into the fragment area; then the DMA of piece t
        (t <= 3) into the raw area, which the conversion's reads have left.
        Piece p of a row is its bytes 128 p .. +127 (k-steps 2 p and
        2 p + 1); DMA instruction i = 4 qb + 2 kk + j of a piece puts lane
        l's 16 bytes of row 32 qb + l % 32, bytes 128 p + 64 kk + 32 (l / 32)
        + 16 j, at raw + 1024 i + 16 l."""
        noconv, done = f".Lxl_noconv_{tag}_%=", f".Lxl_piecedone_{tag}_%="
        self.piece_index(tr, toff)
        tr.raw("s_waitcnt lgkmcnt(0)")
        tr.raw(f"s_cmp_eq_u32 s{S_T2}, 0")
        tr.raw(f"s_cbranch_scc1 {noconv}")
        # conversion of piece t - 1, whose DMAs were issued before this
        # step's K/V DMAs (XL_KV_DMAS of them since)
        tr.raw(f"s_waitcnt vmcnt({XL_KV_DMAS})")
        tr.raw(f"s_sub_u32 s{S_T3}, s{S_T2}, 1")
        tr.raw(f"s_lshl_b32 s{S_T3}, s{S_T3}, 11")
        tr.raw(f"v_add_u32 {vr(R + 32)}, %[rawdelta], %[qrd]")
        tr.raw(f"v_add_u32 {vr(R + 33)}, s{S_T3}, %[qrd]")
        for i in range(8):
            tr.raw(f"ds_read_b128 {vrng(R + 4 * i, 4)}, {vr(R + 32)} offset:{1024 * i}")
        frags = []
        for qb in range(2):
            for kk in range(2):
                # this fragment's two reads have returned (LDS operations
                # complete in order)
                tr.raw(f"s_waitcnt lgkmcnt({6 - 2 * (2 * qb + kk)})")
                j0, j1 = R + 4 * (4 * qb + 2 * kk), R + 4 * (4 * qb + 2 * kk + 1)
                w = R + 36 + 4 * (2 * qb + kk)
                srcs = ((j0, j0 + 1), (j0 + 2, j0 + 3), (j1, j1 + 1), (j1 + 2, j1 + 3))
                for x, (a, b) in enumerate(srcs):
                    tr.raw(f"{self.cvt} {vr(w + x)}, {vr(a)}, {vr(b)}")
                frags.append((w, 1024 * (8 * qb + kk)))
        # scale < 0: Q negated (a sign XOR per element); never for the
        # reference's positive scale
        pos = f".Lxl_qpos_{tag}_%="
        tr.raw("s_cmp_eq_u32 %[qsgn], 0")
        tr.raw(f"s_cbranch_scc1 {pos}")
        for w, _ in frags:
            for x in range(4):
                tr.raw(f"v_xor_b32 {vr(w + x)}, %[qsgn], {vr(w + x)}")
        tr.label(pos)
        for w, off in frags:
            tr.raw(f"ds_write_b128 {vr(R + 33)}, {vrng(w, 4)} offset:{off}")
        # (the fragment writes may still be pending at the return: LDS
        # operations complete in order, so every later wait for a younger
        # one waits for them too, and nothing before the next unit reads
        # the fragment area)
        tr.label(noconv)
        # DMA of piece t
        tr.raw(f"s_cmp_ge_u32 s{S_T2}, {XL_PIECES}")
        tr.raw(f"s_cbranch_scc1 {done}")
        tr.raw(f"s_lshl_b32 s{S_T2}, s{S_T2}, 7")
        for qb in range(2):
            for kk in range(2):
                for j in range(2):
                    i = 4 * qb + 2 * kk + j
                    tr.raw(f"s_add_u32 s{S_T3}, s{S_T2}, {64 * kk + 16 * j}")
                    tr.raw(f"v_add_u32 {vr(R + 52 + i)}, s{S_T3}, %[qoff{qb}]")
                    tr.raw(f"s_add_u32 m0, %[rawb], {1024 * i}")
                    tr.raw("s_nop 0")
                    tr.raw(f"buffer_load_dwordx4 {vr(R + 52 + i)}, s[{S_NQ}:{S_NQ + 3}], 0 offen lds")
        tr.label(done)

    def piece_block_q16(self, tr, R, toff, tag):
        """Q stored in the operand type: in step t <= 3 each wave DMAs the
        fragments of k-steps 2 t and 2 t + 1 of its 64 rows straight into
        the fragment area (the fragment layout is the rows' 16-byte chunks:
        lane l of fragment (qb, ks) holds row 32 qb + l % 32, bytes
        32 ks + 16 (l / 32)); nothing to convert.  Their DMAs stay in flight
        past the step's end (step_wait); the next step's end waits for them,
        or, for those of a unit's last step, the next unit's first wait, for
        the tiles issued after them, which its Q reads follow."""
        done = f".Lxl_piecedone_{tag}_%="
        self.piece_index(tr, toff)
        tr.raw(f"s_cmp_ge_u32 s{S_T2}, {XL_PIECES}")
        tr.raw(f"s_cbranch_scc1 {done}")
        tr.raw(f"s_lshl_b32 s{S_T2}, s{S_T2}, 6")
        tr.raw(f"s_lshl_b32 s{S_T3}, s{S_T2}, 5")
        for qb in range(2):
            for kk in range(2):
                i = 2 * qb + kk
                tr.raw(f"s_add_u32 s{S_VCC}, s{S_T2}, {32 * kk}")
                tr.raw(f"v_add_u32 {vr(R + 52 + i)}, s{S_VCC}, %[qoff{qb}]")
                tr.raw(f"s_add_u32 m0, %[qfb], s{S_T3}")
                tr.raw(f"s_add_u32 m0, m0, {1024 * (8 * qb + kk)}")
                tr.raw("s_nop 0")
                tr.raw(f"buffer_load_dwordx4 {vr(R + 52 + i)}, s[{S_NQ}:{S_NQ + 3}], 0 offen lds")
        tr.label(done)

    def epilogue(self, tr, next_v=True):
        """After the last step, once every wave is done with the K/V
        buffers: V(0) of the next unit (next_v), then O / l of the rows as
        whole lines (store_o_row_l's arithmetic: l the sum over the lane
        pair, O * (l == 0 ? 0 : 1 / l) with the correctly rounded
        division), staged in the wave's 8 KiB at %[rawb]."""
        e = tr.emit
        tr.raw("s_barrier")
        if next_v:
            for j, w in enumerate(("nvw0", "nvw1", "nvw2", "rw3")):
                e(Ins(f"s_mov_b32 s{S_V + j}, %[{w}]", "salu"))
            for j in range(4):
                for x in self.dma("v", VBUF[0], j):
                    e(x)
        t = EP_T
        for qb in range(2):
            e(valu(f"v_mov_b32 {vr(X)}, {vr(LH[qb])}", {vr(LH[qb])}, {vr(X)}))
            e(valu(f"v_mov_b32 {vr(Y)}, {vr(LH[qb])}", {vr(LH[qb])}, {vr(Y)}))
            e(Ins(f"v_permlane32_swap_b32 {vr(X)}, {vr(Y)}", "perm", {vr(X), vr(Y)}, {vr(X), vr(Y)}))
            lv, d, r, n, q, er, inv = (vr(t[0]), vr(t[1]), vr(t[2]), vr(t[3]), vr(t[4]), vr(t[5]),
                                       vr(EP_INV[qb]))
            e(valu(f"v_add_f32 {lv}, {vr(X)}, {vr(Y)}", {vr(X), vr(Y)}, {lv}))
            e(valu(f"v_div_scale_f32 {d}, s[{S_VCC}:{S_VCC + 1}], {lv}, {lv}, 1.0", {lv}, {d}))
            e(Ins(f"v_rcp_f32 {r}, {d}", "trans", {d}, {r}))
            e(valu(f"v_div_scale_f32 {n}, vcc, 1.0, {lv}, 1.0", {lv}, {n}))
            e(valu(f"v_fma_f32 {q}, -{d}, {r}, 1.0", {d, r}, {q}))
            e(valu(f"v_fma_f32 {r}, {q}, {r}, {r}", {q, r}, {r}))
            e(valu(f"v_mul_f32 {q}, {n}, {r}", {n, r}, {q}))
            e(valu(f"v_fma_f32 {er}, -{d}, {q}, {n}", {d, q, n}, {er}))
            e(valu(f"v_fma_f32 {q}, {er}, {r}, {q}", {er, r, q}, {q}))
            e(valu(f"v_fma_f32 {d}, -{d}, {q}, {n}", {d, q, n}, {d}))
            tr.raw("s_nop 3", 4)
            e(valu(f"v_div_fmas_f32 {d}, {d}, {r}, {q}", {d, r, q}, {d}))
            e(valu(f"v_div_fixup_f32 {inv}, {d}, {lv}, 1.0", {d, lv}, {inv}))
            e(valu(f"v_cmp_neq_f32 vcc, 0, {lv}", {lv}, ()))
            e(valu(f"v_cndmask_b32 {inv}, 0, {inv}, vcc", {inv}, {inv}))
        # lane addresses: staging write (row l % 32, F32 chunk 2 g + l / 32 /
        # 16-bit 8-byte half), staging read (row 8 j + l / 8, chunk l % 8),
        # global row offset ((l / 8) rows, chunk l % 8) per 8-row block
        ln, a0, a1 = vr(EP_LANE), vr(t[6]), vr(t[7])
        e(valu(f"v_mbcnt_lo_u32_b32 {ln}, -1, 0", (), {ln}))
        e(valu(f"v_mbcnt_hi_u32_b32 {ln}, -1, {ln}", {ln}, {ln}))
        e(valu(f"v_and_b32 {a0}, 31, {ln}", {ln}, {a0}))
        e(valu(f"v_mul_u32_u24 {a0}, {XL_PITCH}, {a0}", {a0}, {a0}))
        e(valu(f"v_add_u32 {a0}, %[rawb], {a0}", {a0}, {a0}))
        e(valu(f"v_lshrrev_b32 {a1}, 5, {ln}", {ln}, {a1}))
        e(valu(f"v_lshl_add_u32 {vr(EP_STW)}, {a1}, 4, {a0}", {a1, a0}, {vr(EP_STW)}))
        e(valu(f"v_lshl_add_u32 {vr(EP_STW16)}, {a1}, 3, {a0}", {a1, a0}, {vr(EP_STW16)}))
        e(valu(f"v_lshrrev_b32 {a0}, 3, {ln}", {ln}, {a0}))
        e(valu(f"v_and_b32 {a1}, 7, {ln}", {ln}, {a1}))
        e(valu(f"v_mul_u32_u24 {vr(EP_STR)}, {XL_PITCH}, {a0}", {a0}, {vr(EP_STR)}))
        e(valu(f"v_add_u32 {vr(EP_STR)}, %[rawb], {vr(EP_STR)}", {vr(EP_STR)}, {vr(EP_STR)}))
        e(valu(f"v_lshl_add_u32 {vr(EP_STR)}, {a1}, 4, {vr(EP_STR)}", {a1, vr(EP_STR)}, {vr(EP_STR)}))
        e(valu(f"v_mul_lo_u32 {a0}, %[onb2], {a0}", {a0}, {a0}))
        e(valu(f"v_lshl_add_u32 {vr(EP_OOFF)}, {a1}, 4, {a0}", {a1, a0}, {vr(EP_OOFF)}))
        for k in range(8):
            tr.raw(f"s_mul_i32 s{S_TMP}, %[o8], {k}")
            e(valu(f"v_add_u32 {vr(EP_OROW[k])}, s{S_TMP}, {vr(EP_OOFF)}", {vr(EP_OOFF)}, {vr(EP_OROW[k])}))
        for j, w in enumerate(("ow0", "ow1", "ow2", "rw3")):
            e(Ins(f"s_mov_b32 s{S_K + j}, %[{w}]", "salu"))
        # every MFMA result has settled before the paths below read O
        tr.raw("s_nop 7", 8)
        tr.raw("s_nop 7", 8)
        tr.raw("s_nop 7", 8)
        tr.mfma_w.clear()
        tr.raw("s_cmp_eq_u32 %[ot], 0")
        tr.raw("s_cbranch_scc0 .Lxl_o16_%=")
        tb = copy.deepcopy(tr)
        n0 = len(tb.out)
        self.store_f32(tb)
        tr.out.extend(tb.out[n0:])
        tr.raw("s_branch .Lxl_oend_%=")
        tr.label(".Lxl_o16_%=")
        tr.raw("s_cmp_eq_u32 %[ot], 1")
        tr.raw("s_cbranch_scc0 .Lxl_of16_%=")
        tb = copy.deepcopy(tr)
        n0 = len(tb.out)
        self.store_16(tb, "v_cvt_pk_bf16_f32")
        tr.out.extend(tb.out[n0:])
        tr.raw("s_branch .Lxl_oend_%=")
        tr.label(".Lxl_of16_%=")
        tb = copy.deepcopy(tr)
        n0 = len(tb.out)
        self.store_16(tb, "v_cvt_pk_f16_f32")
        tr.out.extend(tb.out[n0:])
        tr.label(".Lxl_oend_%=")

    def zero_o(self, e, regs):
        """In the persistent kernel's block, O's accumulators cleared for the
        next unit once read (the first unit of a workgroup clears them in
        its prologue)."""
        if not getattr(self, "clear_o", False):
            return
        for r in regs:
            e(Ins(f"v_accvgpr_write_b32 a{r}, 0", "accw", (), {f"a{r}"}))

    def store_f32(self, tr):
        """F32 O: per (query block, 32-column block) the 32 rows' 128-byte
        pieces staged, then read back 8 rows x 128 bytes per instruction and
        stored non-temporal (O is not read again)."""
        e = tr.emit
        for rnd in range(8):
            qb, dblk = divmod(rnd, 4)
            va, rb = 24 + 32 * (rnd % 2), 120 + 16 * (rnd % 2)
            for i in range(16):
                a = f"a{A_O + 64 * qb + 16 * dblk + i}"
                e(Ins(f"v_accvgpr_read_b32 {vr(va + i)}, {a}", "valu", {a}, {vr(va + i)}))
            for i in range(16):
                e(valu(f"v_mul_f32 {vr(va + i)}, {vr(va + i)}, {vr(EP_INV[qb])}", {vr(va + i), vr(EP_INV[qb])},
                       {vr(va + i)}))
            for g in range(4):
                e(Ins(f"ds_write_b128 {vr(EP_STW)}, {vrng(va + 4 * g, 4)} offset:{32 * g}", "lds_wr",
                      vset(va + 4 * g, 4) | {vr(EP_STW)}, ()))
            self.zero_o(e, [A_O + 64 * qb + 16 * dblk + i for i in range(16)])
            for jr in range(4):
                e(Ins(f"ds_read_b128 {vrng(rb + 4 * jr, 4)}, {vr(EP_STR)} offset:{8 * XL_PITCH * jr}", "lds_rd",
                      {vr(EP_STR)}, vset(rb + 4 * jr, 4)))
            for jr in range(4):
                e(Ins(f"buffer_store_dwordx4 {vrng(rb + 4 * jr, 4)}, {vr(EP_OROW[4 * qb + jr])}, s[{S_K}:{S_K + 3}], "
                      f"0 offen offset:{128 * dblk} nt", "vmem", vset(rb + 4 * jr, 4) | {vr(EP_OROW[4 * qb + jr])}, ()))

    def store_16(self, tr, cvt):
        """16-bit O: per (query block, pair of 32-column blocks) the 32 rows'
        128-byte pieces staged, then stored as in store_f32."""
        e = tr.emit
        for rnd in range(4):
            qb, dp = divmod(rnd, 2)
            va, wp, rb = 24 + 32 * (rnd % 2), 88 + 16 * (rnd % 2), 120 + 16 * (rnd % 2)
            for dd in range(2):
                for i in range(16):
                    a = f"a{A_O + 64 * qb + 16 * (2 * dp + dd) + i}"
                    e(Ins(f"v_accvgpr_read_b32 {vr(va + 16 * dd + i)}, {a}", "valu", {a}, {vr(va + 16 * dd + i)}))
            for i in range(32):
                e(valu(f"v_mul_f32 {vr(va + i)}, {vr(va + i)}, {vr(EP_INV[qb])}", {vr(va + i), vr(EP_INV[qb])},
                       {vr(va + i)}))
            self.zero_o(e, [A_O + 64 * qb + 16 * (2 * dp + dd) + i for dd in range(2) for i in range(16)])
            for dd in range(2):
                for g in range(4):
                    for h in range(2):
                        s0 = va + 16 * dd + 4 * g + 2 * h
                        w = wp + 8 * dd + 2 * g + h
                        e(valu(f"{cvt} {vr(w)}, {vr(s0)}, {vr(s0 + 1)}", {vr(s0), vr(s0 + 1)}, {vr(w)}))
            for dd in range(2):
                for g in range(4):
                    w = wp + 8 * dd + 2 * g
                    e(Ins(f"ds_write_b64 {vr(EP_STW16)}, {vrng(w, 2)} offset:{64 * dd + 16 * g}", "lds_wr",
                          vset(w, 2) | {vr(EP_STW16)}, ()))
            for jr in range(4):
                e(Ins(f"ds_read_b128 {vrng(rb + 4 * jr, 4)}, {vr(EP_STR)} offset:{8 * XL_PITCH * jr}", "lds_rd",
                      {vr(EP_STR)}, vset(rb + 4 * jr, 4)))
            for jr in range(4):
                e(Ins(f"buffer_store_dwordx4 {vrng(rb + 4 * jr, 4)}, {vr(EP_OROW[4 * qb + jr])}, s[{S_K}:{S_K + 3}], "
                      f"0 offen offset:{128 * dp} nt", "vmem", vset(rb + 4 * jr, 4) | {vr(EP_OROW[4 * qb + jr])}, ()))

    def build_unit(self, q16=False):
        """The unit block of fa_fwd_xlong64: the loop of build() for one
        unit, whose Q fragments are in the fragment area; the first unit of
        a workgroup (operand first != 0) fetches its own K(0), V(0), K(1),
        later ones find them issued by the previous unit and wait only for
        those (the previous unit's O stores, issued after them, complete in
        issue order)."""
        self.q16 = q16
        self.clear_o = True
        tr = Tracker()
        e = tr.emit
        for qb in range(2):
            e(valu(f"v_mov_b32 {vr(M[qb])}, 0xff800000", (), {vr(M[qb])}))
            e(valu(f"v_mov_b32 {vr(LH[qb])}, 0", (), {vr(LH[qb])}))
        # O = 0: the previous unit's epilogue cleared it; the first unit of a
        # workgroup clears it here
        tr.raw("s_cmp_eq_u32 %[first], 0")
        tr.raw("s_cbranch_scc1 .Lxl_ozero_%=")
        for i in range(128):
            e(Ins(f"v_accvgpr_write_b32 a{A_O + i}, 0", "accw", (), {f"a{A_O + i}"}))
        tr.label(".Lxl_ozero_%=")
        q_reads = [Ins(f"ds_read_b128 {arng(A_Q + 4 * i, 4)}, %[qrd] offset:{1024 * i}", "lds_rd", (),
                       aset(A_Q + 4 * i, 4)) for i in range(16)]
        if not q16:
            # (the previous unit's conversions wrote them and waited)
            for x in q_reads:
                e(x)
        for j, w in enumerate(("kw0", "kw1", "kw2", "rw3")):
            e(Ins(f"s_mov_b32 s{S_K + j}, %[{w}]", "salu"))
        for j, w in enumerate(("vw0", "vw1", "vw2", "rw3")):
            e(Ins(f"s_mov_b32 s{S_V + j}, %[{w}]", "salu"))
        for j, w in enumerate(("nqw0", "nqw1", "nqw2", "rw3")):
            e(Ins(f"s_mov_b32 s{S_NQ + j}, %[{w}]", "salu"))
        tr.raw("s_cmp_eq_u32 %[first], 0")
        tr.raw("s_cbranch_scc1 .Lxl_issued_%=")
        for j in range(4):
            for x in self.dma("k", KBUF[0], j):
                e(x)
        for x in self.advance("k"):
            e(x)
        for j in range(4):
            for x in self.dma("v", VBUF[0], j):
                e(x)
        for x in self.advance("v"):
            e(x)
        for j in range(4):
            for x in self.dma("k", KBUF[1], j):
                e(x)
        for x in self.advance("k"):
            e(x)
        tr.raw("s_waitcnt vmcnt(0)")
        tr.raw("s_branch .Lxl_go_%=")
        tr.label(".Lxl_issued_%=")
        for x in self.advance("k") + self.advance("v") + self.advance("k"):
            e(x)
        tr.raw("s_cmp_eq_u32 %[ot], 0")
        tr.raw("s_cbranch_scc0 .Lxl_w16_%=")
        tr.raw(f"s_waitcnt vmcnt({XL_STORES['f32']})")
        tr.raw("s_branch .Lxl_go_%=")
        tr.label(".Lxl_w16_%=")
        tr.raw(f"s_waitcnt vmcnt({XL_STORES['b16']})")
        tr.label(".Lxl_go_%=")
        if q16:
            # the previous unit's fragment DMAs are older than the stores:
            # the wait above has seen them land
            for x in q_reads:
                e(x)
        tr.raw("s_waitcnt lgkmcnt(0)")
        tr.lds = []
        tr.raw("s_barrier")
        pre, seq = self.qk_stream(KBUF[0], 0)
        for r in pre:
            e(r)
        self.merge(tr, seq, [])
        tr.raw("s_barrier")
        for qb in range(2):
            self.row_max(e, 0, qb, [W_BASE + i for i in range(3)])
            e(valu(f"v_max_f32 {vr(M[qb])}, {vr(M[qb])}, {vr(X)}", {vr(M[qb]), vr(X)}, {vr(M[qb])}))
        for x in self.softmax_half(0, 0, 0, (0, 1), True):
            e(x)
        tr.raw(f"s_mov_b32 s{S_T}, 0")
        tr.label(".Lw64_loop_%=")
        tr.raw(f"s_add_u32 s{S_TMP}, s{S_T}, 2")
        tr.raw(f"s_cmp_lt_u32 s{S_TMP}, %[n]")
        tr.raw(".Lw64_tail_%=".join(["s_cbranch_scc0 ", ""]))
        self.step(tr, 0, False, "a", 0, unit=True)
        self.step(tr, 1, False, "b", 1, unit=True)
        tr.raw(f"s_add_u32 s{S_T}, s{S_T}, 2")
        tr.raw("s_branch .Lw64_loop_%=")
        tr.label(".Lw64_tail_%=")
        tr.raw(f"s_add_u32 s{S_TMP}, s{S_T}, 1")
        tr.raw(f"s_cmp_lt_u32 s{S_TMP}, %[n]")
        tr.raw("s_cbranch_scc0 .Lw64_last0_%=")
        self.step(tr, 0, False, "c", 0, unit=True)
        self.step(tr, 1, True, "d", 1, unit=True)
        tr.raw("s_branch .Lw64_done_%=")
        tr.label(".Lw64_last0_%=")
        # (the tracker goes on from step d's end: step e only adds distance
        # on its own path before the epilogue, whose first reads of O wait
        # out every MFMA result)
        te = copy.deepcopy(tr)
        n0 = len(te.out)
        self.step(te, 0, True, "e", 0, unit=True)
        tr.out.extend(te.out[n0:])
        tr.label(".Lw64_done_%=")
        self.epilogue(tr)
        tr.raw("s_branch .Lxl_end_%=")
        lines = tr.out
        for blk in self.slow:
            lines += blk
        lines.append(".Lxl_end_%=:")
        return lines

    return dict(locals())


for _name, _f in _xl_unit_methods().items():
    setattr(Gen, _name, _f)


def check_registers(lines, s_first=S_FIRST, s_last=S_LAST):
    """Every register named is inside the loop's ranges or an operand."""
    for ln in lines:
        for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b", ln):
            if m.group(1):
                kind, lo, hi = m.group(1), int(m.group(2)), int(m.group(3))
            else:
                kind, lo, hi = m.group(4), int(m.group(5)), int(m.group(5))
            if kind == "v":
                assert 24 <= lo and hi <= V_LAST, ln
            else:
                assert 0 <= lo and hi <= A_LAST, ln
        for m in re.finditer(r"\bs\[?(\d+)", ln):
            assert s_first <= int(m.group(1)) <= s_last + 3, ln


def write_unit(path):
    """kd_fa_xlong64_loop.inc: the unit block of fa_fwd_xlong64."""
    out = ["// Generated by gen_w64_loop.py from this directory; do not edit.",
           "// The per-unit block of fa_fwd_xlong64 (kd_fa_kernel.hip) as inline-asm text.", ""]
    for T, q16 in (("bf16", False), ("f16", False), ("bf16", True), ("f16", True)):
        lines = Gen(T).build_unit(q16)
        check_registers(lines, XL_S_FIRST, XL_S_LAST)
        out.append(f"#define KD_XL64_UNIT_{T.upper()}{'_Q16' if q16 else ''} \\")
        for ln in lines:
            out.append(f'    "{ln}\\n" \\')
        out.append('    ""')
        out.append("")
    out.append("#define KD_XL64_CLOBBERS \\")
    regs = [f'"v{i}"' for i in range(24, V_LAST + 1)] + [f'"a{i}"' for i in range(A_LAST + 1)] + \
           [f'"s{i}"' for i in range(XL_S_FIRST, XL_S_LAST + 1)]
    for k in range(0, len(regs), 16):
        out.append("    " + ", ".join(regs[k:k + 16]) + ", \\")
    out.append('    "vcc", "scc", "m0", "memory"')
    with open(path, "w") as f:
        f.write("\n".join(out) + "\n")


def main(path=None, kpre=2, vpre=2, per1=4, check_at=29, check_spread=True):
    """Writes the loop (path, default kd_fa_w64_loop.inc beside this file)
    and the unit block (kd_fa_xlong64_loop.inc in the same directory)."""
    configure(kpre, vpre, per1, check_at, check_spread)
    here = os.path.dirname(os.path.abspath(__file__))
    path = path or os.path.join(here, "kd_fa_w64_loop.inc")
    write_unit(os.path.join(os.path.dirname(os.path.abspath(path)), "kd_fa_xlong64_loop.inc"))
    out = ["// Generated by gen_w64_loop.py from this directory; do not edit.",
           "// The key loop of fa_fwd_w64 (kd_fa_kernel.hip) as inline-asm text.", ""]
    for T in ("bf16", "f16"):
        lines = Gen(T).build()
        check_registers(lines)
        out.append(f"#define KD_W64_LOOP_{T.upper()} \\")
        for ln in lines:
            out.append(f'    "{ln}\\n" \\')
        out.append('    ""')
        out.append("")
    pre = Gen("bf16").build_pre()
    check_registers(pre)
    out.append("#define KD_W64_PRE \\")
    for ln in pre:
        out.append(f'    "{ln}\\n" \\')
    out.append('    ""')
    out.append("")
    out.append("#define KD_W64_PRE_CLOBBERS \\")
    out.append("    " + ", ".join(f'"s{S_K + j}"' for j in range(4)) + ", " +
               ", ".join(f'"s{S_V + j}"' for j in range(4)) + ', "scc", "m0", "memory"')
    out.append("")
    out.append("#define KD_W64_CLOBBERS \\")
    regs = [f'"v{i}"' for i in range(24, V_LAST + 1)] + [f'"a{i}"' for i in range(A_LAST + 1)] + \
           [f'"s{i}"' for i in range(S_FIRST, S_LAST + 1)]
    for k in range(0, len(regs), 16):
        out.append("    " + ", ".join(regs[k:k + 16]) + ", \\")
    out.append('    "vcc", "scc", "m0", "memory"')
    with open(path, "w") as f:
        f.write("\n".join(out) + "\n")


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description="write the fa_fwd_w64 key loop")
    ap.add_argument("out", nargs="?", default=None)
    ap.add_argument("--kpre", type=int, default=2)
    ap.add_argument("--vpre", type=int, default=2)
    ap.add_argument("--per1", type=int, default=4)
    ap.add_argument("--check-at", type=int, default=29)
    ap.add_argument("--check-spread", action=argparse.BooleanOptionalAction, default=True)
    args = ap.parse_args()
    main(args.out, args.kpre, args.vpre, args.per1, args.check_at, args.check_spread)
