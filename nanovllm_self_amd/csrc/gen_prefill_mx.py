#!/usr/bin/env python3
"""Generator of the MFMA prefill kernel's persistent loop (paged_prefill_mx.hip)
for gfx950.

Writes prefill_mx_asm.inc next to this file: four string-literal macros
(NVS_PREFILL_MX_ASM_PAGED, NVS_PREFILL_MX_ASM_LOCAL, and the _F16 pair for
fp16 elements, which differ only in the MFMA, the packing instruction and
the row-sum limit), each the body of one
inline-asm statement that runs all of a work-group's prefill work: it claims
units from its XCD's counter, decodes each from its plan record, and streams
the units' 64-key tiles through one software pipeline that runs on from one
unit into the next.  Run it after editing this file:
python nanovllm_self_amd/csrc/gen_prefill_mx.py

Per wave: 64 query rows as two 32-row q-blocks (qb), one 64-key tile per
iteration, v_mfma_f32_32x32x16_bf16 (or _f16) throughout:
  S^T[kb][qb] (32 keys x 32 q)  = K . Q^T   16 d-steps x ... = 32 MFMAs
  O^T[n][qb]  (32 d x 32 q)    += V^T . P^T                   32 MFMAs
Iteration j: segment A runs PV of tile j-1 beside the first exponentials of
S_j (and, for a unit's first tile, its row max and the running max);
segment B runs QK of tile j+1 beside the rest of S_j's exponentials, the
bf16 packing of P_j and the row sums, and, once its K operands are read,
reads the first operands of tile j's PV.  K/V operands are read from LDS
into AGPR rings six operands ahead of their MFMAs; tiles are copied HBM ->
LDS by buffer loads that write LDS directly (rows out of range read as
zero): K tile j+2 into K buffer j % 2 and V tile j+1 into V buffer
(g+1) % 3, g counting the work-group's iterations (V tiles rotate through
three buffers so the one segment B reads is complete a whole iteration
before; the V address registers move to the current buffer once an
iteration).

From one unit into the next: the fills of unit u's last two iterations copy
unit u+1's key tiles 0 and 1; u's last iteration reads u+1's query rows (in
the wave's query stage since u began) into the Q^T registers and runs QK^T of
u+1's tile 0 in its segment B; u+1's first iteration runs the PV of u's last
tile in its segment A and, beside the QK^T of its tile 1, normalises u's
output and stores it as bf16 (fp16) rows through the wave's query stage
(v_permlane32_swap_b32 pairs the lane halves' 8-byte pieces into 16-byte
chunks).  The iteration parity runs on across units, so u's last V tile and
u+1's first tiles are in opposite buffers.  A unit of one tile, a unit
without a visible key and the work-group's last unit end the pipeline: the
last PV and the output, then the next unit starts afresh.

Units are claimed three ahead: when unit u starts, wave 0 claims unit u+3
(published in LDS before u's first barrier, read by every wave when u ends)
and every wave loads the plan record of unit u+2 (a vector load into VREC,
one dword a lane), claimed while u-1 ran; the record is decoded by u's last
iteration, beside its MFMAs, into a "bank" VGPR holding one value a lane
(BANK_* lanes).  Banks: BANKN2 (u+2), BANKN (u+1), BANKU (u), BANKP (u-1,
for its output); the values in use at a time are read into SGPRs with
v_readlane.

Register map (fixed; the C++ side binds inputs to it):
  v[0:127]    S_j / S_{j+1}: S[par][kb][qb] = v[64 par + 16 (2 kb + qb) ..]
  v[128:191]  P_j / P_{j-1}: P[par][qb][m] = v[128 + 32 par + 16 qb + 4 m ..]
  v[192:199]  K operand LDS addresses, one per d-step st (K buffer 0, kb 0)
  v[200:207]  V operand LDS addresses, per (d-block n, key half e), in the
              current V buffer (an in-out operand: the loop moves them)
  v[208:211]  fill lane offsets (K and V rows have one stride)
  v[212:215]  query-row copy lane offsets (row groups 0..3)
  v216-217 m_run, v218-219 l_run, v220-221 mask limit, v222 -inf,
  v223 a temporary, v224-231 softmax temporaries,
  v232-239 exponential temporaries, v240 block id, v241-242 row sums,
  v243 claim, v244-245 the previous unit's l, v246 output lane offset,
  v247 (lane % 32) - 4 (lane / 32), v248 constants (BANKC_* lanes),
  v249-251 unit banks (next, current, previous), v252 plan record and,
  decoded over it, the bank of the unit after next, v253-254 unused (left to the compiler for the spill lanes of the code
  before the statement), v255 output staging read address
  a[0:63]     Q^T operands: Q[qb][st] = a[32 qb + 4 st ..]
  a[64:191]   O^T accumulators: O[n][qb] = a[64 + 16 (2 n + qb) ..]
  a[192:223]  V operand ring (8 slots), a[224:255] K operand ring (8 slots)
  s[4:23], s37, s60, s61 inputs, s[24:59] unit state, s[64:99] loop state,
  s100 the current iteration's V buffer (its offset from V buffer 0)
"""
from __future__ import annotations

import os
import sys

# The element type of Q, K, V, P and the output: bf16, or fp16 (an fp16
# cache).  set_element() switches the MFMA, the packing of P and of the
# output, and the row-sum limit.
MF = "v_mfma_f32_32x32x16_bf16"
CVT = "v_cvt_pk_bf16_f32"


def set_element(f16):
    global MF, CVT, SUM_LIMIT
    MF = "v_mfma_f32_32x32x16_f16" if f16 else "v_mfma_f32_32x32x16_bf16"
    CVT = "v_cvt_pk_f16_f32" if f16 else "v_cvt_pk_bf16_f32"
    SUM_LIMIT = SUM_LIMIT_F16 if f16 else SUM_LIMIT_BF16


# ----------------------------------------------------------- register map
def S(par, kb, qb):
    b = 64 * par + 16 * (2 * kb + qb)
    return f"v[{b}:{b + 15}]"


def Sr(par, kb, qb, v):
    return f"v{64 * par + 16 * (2 * kb + qb) + v}"


def P(par, qb, m):
    b = 128 + 32 * par + 16 * qb + 4 * m
    return f"v[{b}:{b + 3}]"


def Pr(par, qb, m, e):
    return f"v{128 + 32 * par + 16 * qb + 4 * m + e}"


def Q(qb, st):
    b = 32 * qb + 4 * st
    return f"a[{b}:{b + 3}]"


def O(n, qb):
    b = 64 + 16 * (2 * n + qb)
    return f"a[{b}:{b + 15}]"


def VSLOT(s):
    b = 192 + 4 * s
    return f"a[{b}:{b + 3}]", f"a[{b}:{b + 1}]", f"a[{b + 2}:{b + 3}]"


def KSLOT(s):
    b = 224 + 4 * s
    return f"a[{b}:{b + 3}]"


KADDR = [f"v{192 + st}" for st in range(8)]
VADDR = {(n, e): f"v{200 + 2 * n + e}" for n in range(4) for e in range(2)}
DMAK = [f"v{208 + i}" for i in range(4)]  # K and V fills (equal row strides)
QLANE = [f"v{212 + i}" for i in range(4)]  # query rows 4 i + lane / 16 (+ 16: soffset)
MRUN = ["v216", "v217"]
LRUN = ["v218", "v219"]
LIM = ["v220", "v221"]
NINF = "v222"
TMPV = "v223"
MX = ["v224", "v225"]
SW = ["v226", "v227"]
NMS = ["v228", "v229"]
AL = ["v230", "v231"]
ET = [f"v{232 + i}" for i in range(8)]
BLKV = "v240"
X3 = ["v241", "v242"]  # third partial row sum
CLAIM = "v243"       # the claimed counter value (wave 0, lane 0)
LPREV = ["v244", "v245"]  # l of the previous unit's rows (both key halves)
OOFF = "v246"        # output lane offset: (lane / 16) x row stride + 16 (lane % 16)
LANEC = "v247"       # (lane % 32) - 4 (lane / 32): the mask limit's lane part
BANKC = "v248"       # call constants, lane BANKC_*
BANKN, BANKU, BANKP = "v249", "v250", "v251"  # unit descriptors, lane BANK_*
VREC = "v252"        # plan record of the unit after next, dword k in lane k
BANKN2 = VREC        # the unit after next, decoded over its plan record (read first)
RL = "v255"          # query stage read address of output row lane / 16, chunk lane % 16

# BANKC lanes: call (and wave) constants
BANKC_HGS, BANKC_HPI, BANKC_G, BANKC_HQ1 = 0, 1, 2, 3  # head groups - 1, heads/item, group, Hq - 1
BANKC_CHIN = (4, 5)   # q-block qb's head within the item: (2 w + qb) % hpi
BANKC_CPQ = (6, 7)    # q-block qb's first position in the item: 32 ((2 w + qb) / hpi)
BANKC_KC = (8, 9)     # key base (cache, or the local k), lo / hi
BANKC_VC = (10, 11)
BANKC_KRTS = 12       # local mode: bytes between k (and v) rows; 0 paged
BANKC_KHS, BANKC_VHS = 13, 14  # bytes between kv heads of K and of V
BANKC_Q = (15, 16)
BANKC_QRTS, BANKC_QHS = 17, 18
BANKC_OUT = (19, 20)
BANKC_ORTS, BANKC_OHS = 21, 22
BANKC_BT = (23, 24)   # block tables (paged)
BANKC_BTS = 25        # bytes between block-table rows

# bank lanes: a unit's descriptor
BANK_EX, BANK_NT, BANK_JM, BANK_KF = 0, 1, 2, 3
BANK_KB, BANK_VB = (4, 5), (6, 7)
BANK_RBT = (8, 9, 10)     # block-table row: lo, hi, bytes
BANK_BLK = (11, 12, 13)   # block ids of tiles 0, 1, 2
BANK_LIMB = (14, 15)      # q-block qb: first position + K - L
BANK_OB = ((16, 17, 18), (19, 20, 21))  # output rows of q-block qb: lo, hi, bytes
BANK_QB = ((22, 23, 24), (25, 26, 27))  # query rows of q-block qb: lo, hi, bytes
BANK_NK = ((28, 29, 32), (30, 31, 33))  # key tiles 0, 1: lo, hi, bytes

# scalar inputs (the call's)
S_KROW = S_VROW = "s4"  # bytes between key (and value) rows
S_BS, S_NB, S_M0W, S_SCALE, S_WID = "s5", "s6", "s7", "s8", "s9"
S_CNT = "s[10:11]"   # the XCD's unit counter
S_QST = "s12"        # LDS address of the wave's query stage
S_QD = "s13"         # query stage minus K buffer 0: offset added to K operand addresses
S_XCD, S_NUNITS = "s14", "s15"
S_MPE, S_PE = "s16", "s17"  # units per list entry and ceil(2^32 / it)
S_REC_LO, S_REC_HI = "s18", "s19"  # plan records
S_Q16 = "s20"        # 16 query rows in bytes
S_SLOT = "s21"       # LDS address of claim slot 0 (slot 1: + 4)
S_U0, S_U1 = "s22", "s23"  # the work-group's first two units
S_PE1 = "s37"        # all ones when there is one unit per list entry, else 0
# the next unit
S_NK = [("s24", "s25"), ("s26", "s27")]  # its key tiles 0, 1 (first byte)
S_NREC = ["s28", "s29"]  # their bytes (0: none)
S_NNT, S_NEX = "s30", "s31"  # its tiles; whether it exists
# unit control
S_FLAGS = "s34"      # bit 0: the current unit chains into the next
S_IT = "s35"         # units begun: claim slot S_IT % 2
S_U2 = "s36"         # the unit after next
# the current unit
S_KBASE, S_VBASE = "s[40:41]", "s[42:43]"
S_KBASE_LO, S_KBASE_HI, S_VBASE_LO, S_VBASE_HI = "s40", "s41", "s42", "s43"
S_RBT = "s[44:47]"   # buffer resource of the sequence's block-table row (paged)
S_RBT_W = ["s44", "s45", "s46", "s47"]
S_RBT_NREC = "s46"
S_K, S_NT, S_JM = "s48", "s49", "s50"  # key rows the fills read, tiles, first masked tile
S_BLK012 = ["s51", "s52", "s53"]  # block ids of tiles 0, 1, 2 (paged)
S_RREC = "s[56:59]"  # buffer resource of a plan record
S_RREC_W = ["s56", "s57", "s58", "s59"]
# loop state
S_J, S_LAST = "s64", "s65"
S_B = ["s66", "s67", "s68"]        # block ids of tiles j, j+1, j+2 (paged)
S_ROW = ["s69", "s70", "s71"]      # first cache row of tiles j, j+1, j+2
S_KOFF, S_LB = "s72", "s73"        # key offset in block / logical block of the next block-id read
S_RK, S_RV = "s[76:79]", "s[80:83]"  # buffer resources of the K and V fills
S_RK_W = ["s76", "s77", "s78", "s79"]
S_RV_W = ["s80", "s81", "s82", "s83"]
S_F0, S_F1 = "s[84:85]", "s[86:87]"
S_F0_W = ["s84", "s85"]
S_NEED = ["s[94:95]", "s[96:97]"]  # per q-block lane masks (temporaries)
S_MINF = "s[98:99]"  # lanes whose running max is still -inf (no visible key yet)
S_T = ["s88", "s89", "s90", "s91"]
S_TMP = "s92"
S_BOK = "s93"  # 1 if the block-id load in flight is of a block of the sequence
# temporaries of the unit decode (loop state that is dead between units)
# (not S_MINF, which a chaining last iteration still reads after the decode)
DT = ["s76", "s77", "s78", "s79", "s80", "s81", "s82", "s83", "s84", "s85", "s86", "s87",
      "s88", "s89", "s90", "s91", "s94", "s95", "s96", "s97", "s74", "s75", "s38", "s39"]
S_U2IN = "s60"       # input: the work-group's third unit
S_O4 = "s61"         # 4 output rows in bytes

LDS_V0 = 32768      # V buffer 0 (K buffers at 0 and 16384; V buffers 1 and 2 follow)
TILE = 16384        # bytes of one 64-key bf16 tile
NVBUF = 3           # V buffers: the tile of iteration g in buffer g % 3
S_VB = "s100"       # offset from V buffer 0 of the buffer of the current iteration's tile
BANK_NV0 = (34, 35)  # the unit's value tile 0: lo, hi (its bytes are key tile 0's)
RSRC_W3 = "0x20000"  # raw buffer: 32-bit data format, no swizzle, no stride


PAIR_WAITS = True  # one lgkmcnt wait for each pair of K or V operands
FILL_SLOTS = 24  # segment A slots the fills' set-up and loads are spread over
V_FILL_FIRST = False  # the V fill's loads ahead of the K fill's tile rows


class Emitter:
    def __init__(self):
        self.lines = []
        self.lds = []  # outstanding LDS ops, oldest first (tags)

    def __call__(self, s):
        self.lines.append(s)

    def lds_issue(self, tag, ins):
        self.lines.append(ins)
        self.lds.append(tag)

    def lds_wait(self, tag):
        """Wait until the LDS op `tag` has completed (LDS returns in order).
        With PAIR_WAITS, the wait for an even operand covers the odd one
        after it when that was read too: one wait a pair of operands."""
        if PAIR_WAITS and tag[0] in ("v", "k") and tag[1] % 2 == 0:
            nxt = (tag[0], tag[1] + 1) + tag[2:]
            if nxt in self.lds:
                tag = nxt
        if tag not in self.lds:
            return
        i = self.lds.index(tag)
        after = len(self.lds) - i - 1
        self.lines.append(f"s_waitcnt lgkmcnt({min(after, 15)})")
        self.lds = self.lds[i + 1:]

    def lds_drain(self):
        if self.lds:
            self.lines.append("s_waitcnt lgkmcnt(0)")
        self.lds = []


# ------------------------------------------------------------- VALU lists
# the row sums of a tile may reach SUM_LIMIT before the running max moves:
# no exponential of a tile exceeds 2^16 times the row's running max term.
# fp16 P holds at most 65504: its limit is 2^15.
SUM_LIMIT_BF16 = "0x47800000"  # 65536.0
SUM_LIMIT_F16 = "0x47000000"  # 32768.0
SUM_LIMIT = SUM_LIMIT_BF16


def row_max(par):
    """MX[qb] = scale * (max of the lane's row over the tile's 64 keys), as
    instruction strings.  Independent chains are interleaved so no
    instruction reads the result of the one just before it; two wait states
    separate the VALU writes from the permlane that reads them."""
    it = []
    chains = [(qb, kb, MX[qb] if kb == 0 else SW[qb]) for qb in range(2) for kb in range(2)]
    regs = {(qb, kb): [Sr(par, kb, qb, v) for v in range(16)] for qb in range(2) for kb in range(2)}
    for qb, kb, dst in chains:
        r = regs[(qb, kb)]
        it.append(f"v_max3_f32 {dst}, {r[0]}, {r[1]}, {r[2]}")
    for k in range(3, 15, 2):
        for qb, kb, dst in chains:
            r = regs[(qb, kb)]
            it.append(f"v_max3_f32 {dst}, {dst}, {r[k]}, {r[k + 1]}")
    for qb, kb, dst in chains:
        it.append(f"v_max_f32 {dst}, {dst}, {regs[(qb, kb)][15]}")
    for qb in range(2):
        it.append(f"v_max_f32 {MX[qb]}, {MX[qb]}, {SW[qb]}")
    for qb in range(2):
        it.append(f"v_mov_b32 {SW[qb]}, {MX[qb]}")
    it.append("s_nop 1")
    for qb in range(2):
        it.append(f"v_permlane32_swap_b32 {MX[qb]}, {SW[qb]}")
    for qb in range(2):
        it.append(f"v_max_f32 {MX[qb]}, {MX[qb]}, {SW[qb]}")
    for qb in range(2):
        it.append(f"v_mul_f32 {MX[qb]}, {S_SCALE}, {MX[qb]}")
    return it


def max_update(first):
    """Running max m <- max(m, MX) (first tile: m <- MX), exponent offset
    NMS = -m (0 where m is -inf, so masked scores give exp2(-inf) = 0), the
    lanes still at -inf in S_MINF and, after the first tile, alpha =
    2^(m_old - m_new) in AL (1 where m is -inf) with l_run *= alpha.  One
    wait state follows each exponential before its reader and two each
    v_cmp before the v_cndmask that reads its mask."""
    it = []
    if not first:
        for qb in range(2):
            it.append(f"v_max_f32 {MX[qb]}, {MX[qb]}, {MRUN[qb]}")
        for qb in range(2):
            it.append(f"v_sub_f32 {AL[qb]}, {MRUN[qb]}, {MX[qb]}")
    for qb in range(2):
        it.append(f"v_cmp_eq_f32_e64 {S_NEED[qb]}, {NINF}, {MX[qb]}")
    if not first:
        for qb in range(2):
            it.append(f"v_exp_f32 {AL[qb]}, {AL[qb]}")
    for qb in range(2):
        it.append(f"v_mov_b32 {MRUN[qb]}, {MX[qb]}")
    for qb in range(2):
        it.append(f"v_xor_b32 {NMS[qb]}, 0x80000000, {MX[qb]}")
    for qb in range(2):
        it.append(f"v_cndmask_b32_e64 {NMS[qb]}, {NMS[qb]}, 0, {S_NEED[qb]}")
    if not first:
        for qb in range(2):
            it.append(f"v_cndmask_b32_e64 {AL[qb]}, {AL[qb]}, 1.0, {S_NEED[qb]}")
        for qb in range(2):
            it.append(f"v_mul_f32 {LRUN[qb]}, {LRUN[qb]}, {AL[qb]}")
    it.append(f"s_or_b64 {S_MINF}, {S_NEED[0]}, {S_NEED[1]}")
    return it


def exp_pairs(par):
    """(qb, src_a, src_b, dst P reg) for the 32 bf16 pairs of P_j: P^T slice
    m of q-block qb holds S[m // 2][qb] registers 8 (m % 2) .. + 7."""
    out = []
    for qb in range(2):
        for m in range(4):
            for e in range(4):
                v = 8 * (m % 2) + 2 * e
                out.append((qb, Sr(par, m // 2, qb, v), Sr(par, m // 2, qb, v + 1), Pr(par, qb, m, e)))
    return out


def exp_items(pairs, k0, touched):
    """Exponentials of the pairs in groups of four: eight FMAs, eight
    exponentials, four bf16 packs, then the tile's row sums in fp32 (the
    values before rounding, as a flash softmax keeps its row sum): the
    eight values of a group go into two of the three partial sums (SW, MX,
    X3) in turn; a partial's first write of the tile is a move.
    `touched` collects (qb, partial) across the calls of one tile.  Each
    instruction's operands were written at least two instructions earlier
    (v_dot2c, which would sum the packed values, shares the matrix pipe and
    stalls the MFMAs)."""
    it = []
    for g0 in range(0, len(pairs), 4):
        grp = pairs[g0:g0 + 4]
        qb = grp[0][0]
        assert all(x[0] == qb for x in grp) and len(grp) == 4
        t = [(ET[2 * k], ET[2 * k + 1]) for k in range(len(grp))]
        for k, (_, a, b, p) in enumerate(grp):
            it.append(f"v_fma_f32 {t[k][0]}, {a}, {S_SCALE}, {NMS[qb]}")
            it.append(f"v_fma_f32 {t[k][1]}, {b}, {S_SCALE}, {NMS[qb]}")
        for k in range(len(grp)):
            it.append(f"v_exp_f32 {t[k][0]}, {t[k][0]}")
            it.append(f"v_exp_f32 {t[k][1]}, {t[k][1]}")
        for k, (_, a, b, p) in enumerate(grp):
            it.append(f"{CVT} {p}, {t[k][0]}, {t[k][1]}")
        # t0 + t1 -> t0, t2 + t3 -> t2, ... then two partial sums
        for k in range(len(grp)):
            it.append(f"v_add_f32 {t[k][0]}, {t[k][0]}, {t[k][1]}")
        it.append(f"v_add_f32 {t[0][0]}, {t[0][0]}, {t[1][0]}")
        it.append(f"v_add_f32 {t[2][0]}, {t[2][0]}, {t[3][0]}")
        for m, src in enumerate((t[0][0], t[2][0])):
            j = (k0 + g0 + m) % 3
            acc = (SW[qb], MX[qb], X3[qb])[j]
            if (qb, j) in touched:
                it.append(f"v_add_f32 {acc}, {acc}, {src}")
            else:
                touched.add((qb, j))
                it.append(f"v_mov_b32 {acc}, {src}")
    return it


def tile_sum_items():
    """SW[qb] <- the tile's row sum of the lane (the three partials)."""
    it = [f"v_add_f32 {SW[qb]}, {SW[qb]}, {MX[qb]}" for qb in range(2)]
    it += [f"v_add_f32 {SW[qb]}, {SW[qb]}, {X3[qb]}" for qb in range(2)]
    return it


def cost(ins):
    """Issue cycles of an instruction beside MFMAs (measured on gfx950)."""
    if isinstance(ins, list):
        return sum(cost(x) for x in ins)
    if ins.startswith("v_exp"):
        return 8
    if ins.startswith("s_nop"):
        return 1 + int(ins.split()[1])
    if ins.startswith("buffer_"):
        return 8
    if ins.startswith("s_"):
        return 2
    return 4


def spread(items, slots):
    """Distribute items over `slots` MFMA slots by cumulative cost."""
    total = sum(cost(i) for i in items)
    out = [[] for _ in range(slots)]
    acc, k = 0.0, 0
    per = total / slots if slots else 0
    for s in range(slots):
        target = per * (s + 1)
        while k < len(items) and (acc + cost(items[k]) / 2 <= target or s == slots - 1):
            out[s].append(items[k])
            acc += cost(items[k])
            k += 1
    return out


# ------------------------------------------------------------ LDS reads
def v_read(em, i):
    """V operand i (m = i // 4, n = i % 4) into ring slot i % 8, from the V
    buffer the VADDR registers point at (they move with the iterations)."""
    m, n = divmod(i, 4)
    _, lo, hi = VSLOT(i % 8)
    off = 4096 * m
    em.lds_issue(("v", i, 0), f"ds_read_b64_tr_b16 {lo}, {VADDR[(n, 0)]} offset:{off}")
    em.lds_issue(("v", i, 1), f"ds_read_b64_tr_b16 {hi}, {VADDR[(n, 1)]} offset:{off}")


def early_tags():
    """The LDS reads outstanding when an iteration with a PV starts: the
    first AHEAD V operands, read by the iteration before."""
    return [("v", i, e) for i in range(AHEAD) for e in (0, 1)]


def v_rotate_items():
    """VADDR from the previous iteration's V buffer to the current one's
    (S_VB): + TILE, or - 2 TILE from buffer 2 back to buffer 0.  The SCC
    pair and its move stay together."""
    return [[f"s_mov_b32 {S_TMP}, {TILE}", f"s_cmp_eq_u32 {S_VB}, 0",
             f"s_cselect_b32 {S_TMP}, {-2 * TILE & 0xffffffff:#x}, {S_TMP}"]] + \
        [f"v_add_u32 {VADDR[(n, e)]}, {S_TMP}, {VADDR[(n, e)]}" for n in range(4) for e in range(2)]


def vb_advance(em):
    """S_VB to the next iteration's V buffer."""
    em(f"s_add_u32 {S_VB}, {S_VB}, {TILE}")
    em(f"s_cmp_eq_u32 {S_VB}, {NVBUF * TILE}")
    em(f"s_cselect_b32 {S_VB}, 0, {S_VB}")


def k_read(em, par_buf, i):
    """K operand i (st = i // 2, kb = i % 2) of K buffer par_buf into ring slot i % 8."""
    st, kb = divmod(i, 2)
    off = TILE * par_buf + 8192 * kb
    em.lds_issue(("k", i), f"ds_read_b128 {KSLOT(i % 8)}, {KADDR[st]} offset:{off}")


def pv_mfmas(em, i, ppar):
    m, n = divmod(i, 4)
    slot = VSLOT(i % 8)[0]
    return [f"{MF} {O(n, qb)}, {slot}, {P(ppar, qb, m)}, {O(n, qb)}" for qb in range(2)]


def qk_mfmas(i, spar):
    st, kb = divmod(i, 2)
    slot = KSLOT(i % 8)
    return [f"{MF} {S(spar, kb, qb)}, {slot}, {Q(qb, st)}, {S(spar, kb, qb) if st else 0}" for qb in range(2)]


AHEAD = 6  # operands read ahead of their MFMAs (at most 7: the rings hold 8)
NA = 12  # exponential pairs of segment A


def read_ahead_a(em, spar, i, last=False):
    """Segment A's read-ahead after PV operand i: V operand i + AHEAD, or,
    in the last AHEAD slots, the first K operands of segment B (none in a
    unit's last iteration, whose segment B has no QK^T)."""
    if i + AHEAD < 16:
        v_read(em, i + AHEAD)
    elif not last:
        k_read(em, spar, i + AHEAD - 16)

# Optional callback mark(em, k) at the phase boundaries of an iteration
# (k = 0 after the tile rows, 1 after segment A, 2 after segment B, 3 after
# the fills' wait, 4 after the barrier), after the prologue (5), at the end
# (6) and mark(em, None) at the start of the program; None in the product.
MARK = None


def mark(em, k):
    if MARK is not None:
        MARK(em, k)


# ------------------------------------------------------------------ fills
def fill_tile(paged, which, row, tile, blk, par_dst, nxt=None, tile_add=0):
    """Instructions that copy one 64-key tile (K or V) into LDS: a K tile
    into K buffer par_dst, a V tile into the V buffer after S_VB's (the
    next iteration's).  row = first cache row of the tile (SGPR), tile =
    SGPR holding its index less tile_add (for the row count), blk = its
    block id (paged; < 0: missing).  nxt = "sel": tile index ntiles is the
    next unit's key tile 0 instead; "one": the next unit's key tile 1;
    "v0": the next unit's value tile 0 (read from its bank).  Returns a
    list whose items are instruction strings or groups (lists) that must
    stay together: each m0 write, its wait state and its direct-to-LDS
    load, each SCC write with its readers, and each lane read with the wait
    states before its loads."""
    base_lo, base_hi = (S_KBASE_LO, S_KBASE_HI) if which == "k" else (S_VBASE_LO, S_VBASE_HI)
    rowb = S_KROW if which == "k" else S_VROW
    rs = S_RK_W if which == "k" else S_RV_W
    rsrc = S_RK if which == "k" else S_RV
    offs = DMAK
    t0 = S_T[0] if which == "k" else S_T[1]
    out = [
        f"s_mul_i32 {rs[0]}, {row}, {rowb}",
        f"s_mul_hi_u32 {rs[1]}, {row}, {rowb}",
        f"s_add_u32 {rs[0]}, {rs[0]}, {base_lo}",
        f"s_addc_u32 {rs[1]}, {rs[1]}, {base_hi}",
        # rows of the tile that hold keys: clamp(K - 64 t, 0, 64)
        f"s_lshl_b32 {t0}, {tile}, 6",
    ]
    if tile_add:
        out.append(f"s_add_u32 {t0}, {t0}, {64 * tile_add}")
    out += [
        f"s_sub_i32 {t0}, {S_K}, {t0}",
        f"s_max_i32 {t0}, {t0}, 0",
        f"s_min_i32 {t0}, {t0}, 64",
        f"s_mul_i32 {rs[2]}, {t0}, {rowb}",
    ]
    if paged:
        out.append([f"s_cmp_lt_i32 {blk}, 0", f"s_cselect_b32 {rs[2]}, 0, {rs[2]}"])
    if nxt == "sel":  # tile index = ntiles: the next unit's tile 0
        out.append([
            f"s_cmp_eq_u32 {tile}, {S_NT}",
            f"s_cselect_b64 s[{rs[0][1:]}:{rs[1][1:]}], s[{S_NK[0][0][1:]}:{S_NK[0][1][1:]}], s[{rs[0][1:]}:{rs[1][1:]}]",
            f"s_cselect_b32 {rs[2]}, {S_NREC[0]}, {rs[2]}",
        ])
    elif nxt == "one":  # the next unit's tile 1, whatever this unit's are
        out = [f"s_mov_b32 {rs[0]}, {S_NK[1][0]}", f"s_mov_b32 {rs[1]}, {S_NK[1][1]}",
               f"s_mov_b32 {rs[2]}, {S_NREC[1]}"]
    elif nxt == "v0":  # the next unit's value tile 0 (as many rows as its key tile 0)
        out = [[f"v_readlane_b32 {rs[0]}, {BANKN}, {BANK_NV0[0]}",
                f"v_readlane_b32 {rs[1]}, {BANKN}, {BANK_NV0[1]}", "s_nop 4"],
               f"s_mov_b32 {rs[2]}, {S_NREC[0]}"]
    out.append(f"s_and_b32 {rs[1]}, {rs[1]}, 0xffff")
    out.append(f"s_mov_b32 {rs[3]}, {RSRC_W3}")
    if which == "k":
        for i in range(4):
            out.append([f"s_add_u32 m0, {S_M0W}, {TILE * par_dst + 1024 * i}", "s_nop 0",
                        f"buffer_load_dwordx4 {offs[i]}, {rsrc}, 0 offen lds"])
    else:
        vb = S_T[3]  # the V buffer after S_VB's, + the wave's rows
        out += [[f"s_add_u32 {vb}, {S_VB}, {TILE}", f"s_cmp_eq_u32 {vb}, {NVBUF * TILE}",
                 f"s_cselect_b32 {vb}, 0, {vb}"], f"s_add_u32 {vb}, {vb}, {S_M0W}"]
        for i in range(4):
            out.append([f"s_add_u32 m0, {vb}, {LDS_V0 + 1024 * i}", "s_nop 0",
                        f"buffer_load_dwordx4 {offs[i]}, {rsrc}, 0 offen lds"])
    return out


def emit_items(em, items):
    for x in items:
        if isinstance(x, list):
            for y in x:
                em(y)
        else:
            em(x)


def block_row(em, dst_row, blk):
    """Cache row of the tile whose block id is in blk and key offset S_KOFF."""
    em(f"s_max_i32 {S_T[2]}, {blk}, 0")
    em(f"s_mul_i32 {dst_row}, {S_T[2]}, {S_BS}")
    em(f"s_add_u32 {dst_row}, {dst_row}, {S_KOFF}")


def advance_tile(em):
    """(S_KOFF, S_LB) to the next 64-key tile."""
    em(f"s_add_u32 {S_KOFF}, {S_KOFF}, 64")
    em(f"s_cmp_eq_u32 {S_KOFF}, {S_BS}")
    em(f"s_cselect_b32 {S_KOFF}, 0, {S_KOFF}")
    em(f"s_cselect_b32 {S_T[3]}, 1, 0")
    em(f"s_add_u32 {S_LB}, {S_LB}, {S_T[3]}")


def tile_rows_items(paged, first):
    """The fills' tile j+2, as items for the slots of segment A: its block id
    (paged: from the record for a first tile, else taken from the load of
    the iteration before) and cache row, S_KOFF and S_LB moved on, and the
    load of tile j+3's block id issued (in place in BLKV); then S_T[2] =
    j + 2.  Each SCC pair, and the lane read with its wait state, is a
    group."""
    it = []
    if paged:
        d = S_B[2]
        if first:
            it.append(f"s_mov_b32 {d}, {S_BLK012[2]}")
        else:
            it.append([f"v_readfirstlane_b32 {d}, {BLKV}", "s_nop 0", f"s_cmp_lt_u32 {d}, {S_NB}",
                       f"s_cselect_b32 {d}, {d}, -1"])
            it.append([f"s_cmp_eq_u32 {S_BOK}, 0", f"s_cselect_b32 {d}, -1, {d}"])
        it += [f"s_max_i32 {S_T[2]}, {d}, 0", f"s_mul_i32 {S_ROW[2]}, {S_T[2]}, {S_BS}",
               f"s_add_u32 {S_ROW[2]}, {S_ROW[2]}, {S_KOFF}"]
        it.append([f"s_add_u32 {S_KOFF}, {S_KOFF}, 64", f"s_cmp_eq_u32 {S_KOFF}, {S_BS}",
                   f"s_cselect_b32 {S_KOFF}, 0, {S_KOFF}", f"s_cselect_b32 {S_T[3]}, 1, 0"])
        it += [f"s_add_u32 {S_LB}, {S_LB}, {S_T[3]}", f"s_lshl_b32 {S_T[2]}, {S_LB}, 2",
               f"v_mov_b32 {BLKV}, {S_T[2]}", f"buffer_load_dword {BLKV}, {BLKV}, {S_RBT}, 0 offen"]
        it.append([f"s_cmp_lt_u32 {S_T[2]}, {S_RBT_NREC}", f"s_cselect_b32 {S_BOK}, 1, 0"])
    else:
        it += [f"s_add_u32 {S_T[2]}, {S_J}, 2", f"s_lshl_b32 {S_ROW[2]}, {S_T[2]}, 6"]
    it.append(f"s_add_u32 {S_T[2]}, {S_J}, 2")
    return it


# ----------------------------------------------------------------- blocks
def claim(em, lbl):
    """Wave 0, lane 0 claims a unit for the work-group: an atomic add of 1 on
    the XCD's counter whose old value lands in CLAIM while the unit's first
    iteration runs (its wait on vmcnt completes it; every other lane and
    wave gets 0)."""
    em(f"v_mov_b32 {CLAIM}, 0")
    em(f"s_cmp_lg_u32 {S_WID}, 0")
    em(f"s_cbranch_scc1 {lbl}claimed")
    em(f"s_mov_b64 {S_F0}, exec")
    em("s_mov_b64 exec, 1")
    em(f"v_mov_b32 {ET[0]}, 0")
    em(f"v_mov_b32 {ET[1]}, 1")
    em("s_nop 4")
    em(f"global_atomic_add {CLAIM}, {ET[0]}, {ET[1]}, {S_CNT} sc0")
    em(f"s_mov_b64 exec, {S_F0}")
    em(f"{lbl}claimed:")


def slot_address(em_or_list, dst_v):
    """dst_v <- LDS address of the claim slot of the current unit (S_IT % 2)."""
    ins = [f"s_and_b32 {S_TMP}, {S_IT}, 1", f"s_lshl_b32 {S_TMP}, {S_TMP}, 2",
           f"s_add_u32 {S_TMP}, {S_TMP}, {S_SLOT}", f"v_mov_b32 {dst_v}, {S_TMP}"]
    for x in ins:
        em_or_list(x)


def claim_publish(em, lbl):
    """Wave 0 writes the claim it made into the current unit's claim slot;
    the barrier that follows makes it visible to the other waves."""
    em(f"s_cmp_lg_u32 {S_WID}, 0")
    em(f"s_cbranch_scc1 {lbl}pub")
    slot_address(em, ET[0])
    em(f"s_mov_b64 {S_F0}, exec")
    em("s_mov_b64 exec, 1")
    em("s_nop 4")
    em(f"ds_write_b32 {ET[0]}, {CLAIM}")
    em(f"s_mov_b64 exec, {S_F0}")
    em(f"{lbl}pub:")
    em("s_waitcnt lgkmcnt(0)")


def divmod_pe(q, r, u, t):
    """q, r <- u / units-per-entry, u % units-per-entry: a high multiply by
    ceil(2^32 / PE) (0 when PE = 1, where S_PE1 adds u itself), exact or one
    too large, corrected by the remainder's sign.  Uses no SCC across
    instructions."""
    return [
        f"s_mul_hi_u32 {q}, {u}, {S_MPE}",
        f"s_and_b32 {t}, {u}, {S_PE1}",
        f"s_add_u32 {q}, {q}, {t}",
        f"s_mul_i32 {r}, {q}, {S_PE}",
        f"s_sub_i32 {r}, {u}, {r}",
        f"s_ashr_i32 {t}, {r}, 31",
        f"s_add_i32 {q}, {q}, {t}",
        f"s_and_b32 {t}, {t}, {S_PE}",
        f"s_add_i32 {r}, {r}, {t}",
    ]


def record_load_items(u):
    """Vector load of unit u's plan record into VREC (dword k in lane k;
    lanes past 16 read nothing and get 0).  A unit past the list loads
    record 0 (its decode marks it absent)."""
    q, r, t = S_RREC_W[0], S_RREC_W[1], S_RREC_W[2]
    it = divmod_pe(q, r, u, t)
    it += [
        f"s_cmp_lt_u32 {u}, {S_NUNITS}",
        f"s_cselect_b32 {q}, {q}, 0",
        f"s_lshl_b32 {q}, {q}, 6",
        f"s_add_u32 {S_RREC_W[0]}, {q}, {S_REC_LO}",
        f"s_addc_u32 {S_RREC_W[1]}, {S_REC_HI}, 0",
        f"s_and_b32 {S_RREC_W[1]}, {S_RREC_W[1]}, 0xffff",
        f"s_mov_b32 {S_RREC_W[2]}, 64",
        f"s_mov_b32 {S_RREC_W[3]}, {RSRC_W3}",
        # lane offsets 4 x lane, in VREC itself (its last record is decoded)
        f"v_mbcnt_lo_u32_b32 {VREC}, -1, 0",
        f"v_mbcnt_hi_u32_b32 {VREC}, -1, {VREC}",
        f"v_lshlrev_b32 {VREC}, 2, {VREC}",
        f"buffer_load_dword {VREC}, {VREC}, {S_RREC}, 0 offen",
    ]
    return it


class Items(list):
    """Instruction strings collected for a slot schedule (called like an
    emitter)."""

    def __call__(self, ins):
        self.append(ins)


def readlanes(em, pairs):
    """SGPR <- bank lane, for (sgpr, bank, lane) triples; then the wait
    states before a scalar or memory instruction reads them."""
    for sd, bank, lane in pairs:
        em(f"v_readlane_b32 {sd}, {bank}, {lane}")
    em("s_nop 4")


def decode(em, u, paged, bank=None):
    """Unit u (a claimed index) from its plan record in VREC into bank
    (BANKN2).  u = entry x PE + r, r = kv head x head groups + head group."""
    BANKN = bank or BANKN2
    t = list(DT)
    ex, q, r, hkv, hg, tt = t[:6]
    em(f"s_cmp_lt_u32 {u}, {S_NUNITS}")
    em(f"s_cselect_b32 {ex}, 1, 0")
    for x in divmod_pe(q, r, u, hkv):
        em(x)
    em(f"v_readlane_b32 {tt}, {BANKC}, {BANKC_HGS}")
    em("s_nop 4")
    em(f"s_lshr_b32 {hkv}, {r}, {tt}")
    em(f"s_and_b32 {hg}, {r}, {tt}")
    # record fields
    q0, L, blk0, blk1, blk2, p0, nt, kf, off, k0c, b, btb = t[6:18]
    readlanes(em, [(q0, VREC, 1), (L, VREC, 2), (blk0, VREC, 5), (blk1, VREC, 6), (blk2, VREC, 7),
                   (p0, VREC, 8), (nt, VREC, 9), (kf, VREC, 10), (off, VREC, 11), (k0c, VREC, 12),
                   (b, VREC, 13), (btb, VREC, 14)])
    em(f"s_cmp_eq_u32 {ex}, 0")
    em(f"s_cselect_b32 {nt}, 0, {nt}")
    for sv, lane in ((ex, BANK_EX), (nt, BANK_NT), (kf, BANK_KF), (btb, BANK_RBT[2]), (blk0, BANK_BLK[0]),
                     (blk1, BANK_BLK[1]), (blk2, BANK_BLK[2])):
        em(f"v_writelane_b32 {BANKN}, {sv}, {lane}")
    # free: ex, r, tt (btb, blk2 written); reuse them
    c0, c1, c2, c3 = ex, r, tt, btb
    m0, m1 = t[18], t[19]
    # K and V bases: cache (or local k / v) + k0c x row stride + kv head x head stride
    for base, hs, lanes in ((BANKC_KC, BANKC_KHS, BANK_KB), (BANKC_VC, BANKC_VHS, BANK_VB)):
        readlanes(em, [(c0, BANKC, base[0]), (c1, BANKC, base[1]), (c2, BANKC, BANKC_KRTS), (c3, BANKC, hs)])
        em(f"s_mul_i32 {m0}, {k0c}, {c2}")
        em(f"s_mul_hi_u32 {m1}, {k0c}, {c2}")
        em(f"s_add_u32 {c0}, {c0}, {m0}")
        em(f"s_addc_u32 {c1}, {c1}, {m1}")
        em(f"s_mul_i32 {m0}, {hkv}, {c3}")
        em(f"s_mul_hi_u32 {m1}, {hkv}, {c3}")
        em(f"s_add_u32 {c0}, {c0}, {m0}")
        em(f"s_addc_u32 {c1}, {c1}, {m1}")
        em(f"v_writelane_b32 {BANKN}, {c0}, {lanes[0]}")
        em(f"v_writelane_b32 {BANKN}, {c1}, {lanes[1]}")
        kb_lo, kb_hi = (t[20], t[21]) if base == BANKC_KC else (t[22], t[23])
        em(f"s_mov_b32 {kb_lo}, {c0}")
        em(f"s_mov_b32 {kb_hi}, {c1}")
    vb_lo, vb_hi = t[22], t[23]
    kb_lo, kb_hi = t[20], t[21]
    # key tiles 0 and 1 of the unit (what a fill of tile t reads)
    for tl in range(2):
        lo, hi, rec = c0, c1, c2
        blk = blk0 if tl == 0 else blk1
        # rows of the tile that hold keys: clamp(kf - 64 t, 0, 64)
        em(f"s_sub_i32 {rec}, {kf}, {64 * tl}")
        em(f"s_max_i32 {rec}, {rec}, 0")
        em(f"s_min_i32 {rec}, {rec}, 64")
        em(f"s_mul_i32 {rec}, {rec}, {S_KROW}")
        if paged:
            # first row: max(blk, 0) x block size + (64 t) % block size
            em(f"s_max_i32 {m0}, {blk}, 0")
            em(f"s_mul_i32 {m0}, {m0}, {S_BS}")
            if tl == 1:
                em(f"s_cmp_gt_u32 {S_BS}, 64")
                em(f"s_cselect_b32 {m1}, 64, 0")
                em(f"s_add_u32 {m0}, {m0}, {m1}")
            em(f"s_cmp_lt_i32 {blk}, 0")
            em(f"s_cselect_b32 {rec}, 0, {rec}")
        else:
            em(f"s_mov_b32 {m0}, {64 * tl}")
        em(f"s_cmp_eq_u32 {nt}, 0")
        em(f"s_cselect_b32 {rec}, 0, {rec}")
        em(f"s_mul_i32 {lo}, {m0}, {S_KROW}")
        em(f"s_mul_hi_u32 {hi}, {m0}, {S_KROW}")
        em(f"s_add_u32 {lo}, {lo}, {kb_lo}")
        em(f"s_addc_u32 {hi}, {hi}, {kb_hi}")
        em(f"s_and_b32 {hi}, {hi}, 0xffff")
        em(f"v_writelane_b32 {BANKN}, {lo}, {BANK_NK[tl][0]}")
        em(f"v_writelane_b32 {BANKN}, {hi}, {BANK_NK[tl][1]}")
        em(f"v_writelane_b32 {BANKN}, {rec}, {BANK_NK[tl][2]}")
        if tl == 0:  # the value tile 0: the same rows of the value base
            em(f"s_mul_i32 {lo}, {m0}, {S_KROW}")
            em(f"s_mul_hi_u32 {hi}, {m0}, {S_KROW}")
            em(f"s_add_u32 {lo}, {lo}, {vb_lo}")
            em(f"s_addc_u32 {hi}, {hi}, {vb_hi}")
            em(f"v_writelane_b32 {BANKN}, {lo}, {BANK_NV0[0]}")
            em(f"v_writelane_b32 {BANKN}, {hi}, {BANK_NV0[1]}")
    # block-table row: bt + b x row bytes
    readlanes(em, [(c0, BANKC, BANKC_BT[0]), (c1, BANKC, BANKC_BT[1]), (c2, BANKC, BANKC_BTS)])
    em(f"s_mul_i32 {m0}, {b}, {c2}")
    em(f"s_mul_hi_u32 {m1}, {b}, {c2}")
    em(f"s_add_u32 {c0}, {c0}, {m0}")
    em(f"s_addc_u32 {c1}, {c1}, {m1}")
    em(f"s_and_b32 {c1}, {c1}, 0xffff")
    em(f"v_writelane_b32 {BANKN}, {c0}, {BANK_RBT[0]}")
    em(f"v_writelane_b32 {BANKN}, {c1}, {BANK_RBT[1]}")
    # q-blocks: head, position, rows inside the sequence and the group
    hpi, g, hq1 = t[20], t[21], t[22]
    readlanes(em, [(hpi, BANKC, BANKC_HPI), (g, BANKC, BANKC_G), (hq1, BANKC, BANKC_HQ1)])
    limb = []
    for qb in range(2):
        hin, pq, rows, row, hq = c0, c1, c2, c3, m0
        readlanes(em, [(hin, BANKC, BANKC_CHIN[qb]), (pq, BANKC, BANKC_CPQ[qb])])
        em(f"s_mul_i32 {m1}, {hg}, {hpi}")
        em(f"s_add_u32 {hin}, {hin}, {m1}")          # head within the group
        em(f"s_mul_i32 {hq}, {hkv}, {g}")
        em(f"s_add_u32 {hq}, {hq}, {hin}")           # query head
        em(f"s_min_u32 {hq}, {hq}, {hq1}")
        em(f"s_add_u32 {pq}, {pq}, {p0}")            # first position
        em(f"s_add_u32 {m1}, {pq}, {off}")
        em(f"v_writelane_b32 {BANKN}, {m1}, {BANK_LIMB[qb]}")
        limb.append(BANK_LIMB[qb])
        # rows = (hin < g && pq < L) ? min(32, L - pq) : 0; row = q0 + (active ? pq : 0)
        em(f"s_sub_i32 {rows}, {L}, {pq}")
        em(f"s_min_i32 {rows}, {rows}, 32")
        em(f"s_cmp_lt_i32 {pq}, {L}")
        em(f"s_cselect_b32 {rows}, {rows}, 0")
        em(f"s_cselect_b32 {row}, {pq}, 0")
        em(f"s_cmp_lt_u32 {hin}, {g}")
        em(f"s_cselect_b32 {rows}, {rows}, 0")
        em(f"s_cselect_b32 {row}, {row}, 0")
        em(f"s_add_u32 {row}, {row}, {q0}")
        for tensor, rts, hs, lanes in ((BANKC_Q, BANKC_QRTS, BANKC_QHS, BANK_QB[qb]),
                                       (BANKC_OUT, BANKC_ORTS, BANKC_OHS, BANK_OB[qb])):
            lo, hi, rt, hsv = t[23], m1, pq, hin
            # pq and hin are dead now (pq kept in the limit lane)
            readlanes(em, [(lo, BANKC, tensor[0]), (hi, BANKC, tensor[1]), (rt, BANKC, rts), (hsv, BANKC, hs)])
            # lo:hi += row x rts + hq x hs
            x0, x1 = S_TMP, S_RREC_W[3]
            em(f"s_mul_i32 {x0}, {row}, {rt}")
            em(f"s_mul_hi_u32 {x1}, {row}, {rt}")
            em(f"s_add_u32 {lo}, {lo}, {x0}")
            em(f"s_addc_u32 {hi}, {hi}, {x1}")
            em(f"s_mul_i32 {x0}, {hq}, {hsv}")
            em(f"s_mul_hi_u32 {x1}, {hq}, {hsv}")
            em(f"s_add_u32 {lo}, {lo}, {x0}")
            em(f"s_addc_u32 {hi}, {hi}, {x1}")
            em(f"s_and_b32 {hi}, {hi}, 0xffff")
            em(f"s_mul_i32 {x0}, {rows}, {rt}")
            em(f"v_writelane_b32 {BANKN}, {lo}, {lanes[0]}")
            em(f"v_writelane_b32 {BANKN}, {hi}, {lanes[1]}")
            em(f"v_writelane_b32 {BANKN}, {x0}, {lanes[2]}")
    # first tile that some row of the wave does not see whole:
    # max(0, min(pq0, pq1) + K - L + 1) / 64
    em("s_nop 1")
    readlanes(em, [(c0, BANKN, BANK_LIMB[0]), (c1, BANKN, BANK_LIMB[1])])
    em(f"s_min_i32 {c0}, {c0}, {c1}")
    em(f"s_add_i32 {c0}, {c0}, 1")
    em(f"s_max_i32 {c0}, {c0}, 0")
    em(f"s_lshr_b32 {c0}, {c0}, 6")
    em(f"v_writelane_b32 {BANKN}, {c0}, {BANK_JM}")
    em("s_nop 1")


def advance_units(em):
    """Units move on: BANKP <- BANKU <- BANKN <- BANKN2; the current unit's
    values in use and the next unit's key tiles into SGPRs."""
    em(f"v_mov_b32 {BANKP}, {BANKU}")
    em(f"v_mov_b32 {BANKU}, {BANKN}")
    em(f"v_mov_b32 {BANKN}, {BANKN2}")
    em("s_nop 1")
    readlanes(em, [(S_KBASE_LO, BANKU, BANK_KB[0]), (S_KBASE_HI, BANKU, BANK_KB[1]),
                   (S_VBASE_LO, BANKU, BANK_VB[0]), (S_VBASE_HI, BANKU, BANK_VB[1]),
                   (S_K, BANKU, BANK_KF), (S_NT, BANKU, BANK_NT), (S_JM, BANKU, BANK_JM),
                   (S_RBT_W[0], BANKU, BANK_RBT[0]), (S_RBT_W[1], BANKU, BANK_RBT[1]),
                   (S_RBT_W[2], BANKU, BANK_RBT[2]),
                   (S_BLK012[0], BANKU, BANK_BLK[0]), (S_BLK012[1], BANKU, BANK_BLK[1]),
                   (S_BLK012[2], BANKU, BANK_BLK[2]),
                   (S_NEX, BANKN, BANK_EX), (S_NNT, BANKN, BANK_NT),
                   (S_NK[0][0], BANKN, BANK_NK[0][0]), (S_NK[0][1], BANKN, BANK_NK[0][1]),
                   (S_NREC[0], BANKN, BANK_NK[0][2]),
                   (S_NK[1][0], BANKN, BANK_NK[1][0]), (S_NK[1][1], BANKN, BANK_NK[1][1]),
                   (S_NREC[1], BANKN, BANK_NK[1][2])])
    em(f"s_mov_b32 {S_RBT_W[3]}, {RSRC_W3}")


def set_lim(em):
    """The current unit's mask limits: first position of the q-block + K - L
    + (lane % 32) - 4 (lane / 32)."""
    l0, l1 = S_TMP, S_RREC_W[3]
    readlanes(em, [(l0, BANKU, BANK_LIMB[0]), (l1, BANKU, BANK_LIMB[1])])
    em(f"v_add_u32 {LIM[0]}, {l0}, {LANEC}")
    em(f"v_add_u32 {LIM[1]}, {l1}, {LANEC}")


def q_prefetch(em, bank, guard=False):
    """The query rows of the unit in `bank` into the wave's query stage:
    row r of q-block qb at 256 (32 qb + r), its 16-byte chunk c at slot
    c ^ swz(r) (the K tiles' swizzle); rows past the q-block's (resource
    size) read as zero."""
    readlanes(em, [(S_RK_W[0], bank, BANK_QB[0][0]), (S_RK_W[1], bank, BANK_QB[0][1]),
                   (S_RK_W[2], bank, BANK_QB[0][2]),
                   (S_RV_W[0], bank, BANK_QB[1][0]), (S_RV_W[1], bank, BANK_QB[1][1]),
                   (S_RV_W[2], bank, BANK_QB[1][2])])
    em(f"s_mov_b32 {S_RK_W[3]}, {RSRC_W3}")
    em(f"s_mov_b32 {S_RV_W[3]}, {RSRC_W3}")
    if guard:
        em(f"s_cmp_eq_u32 {S_NNT}, 0")
        em(f"s_cselect_b32 {S_RK_W[2]}, 0, {S_RK_W[2]}")
        em(f"s_cselect_b32 {S_RV_W[2]}, 0, {S_RV_W[2]}")
    for qb, rs in ((0, S_RK), (1, S_RV)):
        for i in range(8):
            em(f"s_add_u32 m0, {S_QST}, {1024 * (8 * qb + i)}")
            em("s_nop 0")
            em(f"buffer_load_dwordx4 {QLANE[i % 4]}, {rs}, {0 if i < 4 else S_Q16} offen lds")


def k_prefetch(em, tiles, bank):
    """Key tiles 0 and 1 of a unit into K buffers 0 and 1 and its value tile
    0 into V buffer S_VB (the next iteration's), rows 16 w .. 16 w + 15 of
    each, as the loop's fills: tiles = ((lo, hi, bytes), ...) SGPR names,
    bank = the unit's bank (the value tile's address)."""
    for t, ((lo, hi, rec), rs_w) in enumerate(zip(tiles, (S_RK_W, S_RV_W))):
        em(f"s_mov_b32 {rs_w[0]}, {lo}")
        em(f"s_and_b32 {rs_w[1]}, {hi}, 0xffff")
        em(f"s_mov_b32 {rs_w[2]}, {rec}")
        em(f"s_mov_b32 {rs_w[3]}, {RSRC_W3}")
        rsrc = S_RK if t == 0 else S_RV
        for i in range(4):
            em(f"s_add_u32 m0, {S_M0W}, {TILE * t + 1024 * i}")
            em("s_nop 0")
            em(f"buffer_load_dwordx4 {DMAK[i]}, {rsrc}, 0 offen lds")
    # the value tile: as many rows as key tile 0
    em(f"v_readlane_b32 {S_RK_W[0]}, {bank}, {BANK_NV0[0]}")
    em(f"v_readlane_b32 {S_RK_W[1]}, {bank}, {BANK_NV0[1]}")
    em("s_nop 4")
    em(f"s_and_b32 {S_RK_W[1]}, {S_RK_W[1]}, 0xffff")
    em(f"s_mov_b32 {S_RK_W[2]}, {tiles[0][2]}")
    em(f"s_add_u32 {S_TMP}, {S_VB}, {S_M0W}")
    for i in range(4):
        em(f"s_add_u32 m0, {S_TMP}, {LDS_V0 + 1024 * i}")
        em("s_nop 0")
        em(f"buffer_load_dwordx4 {DMAK[i]}, {S_RK}, 0 offen lds")


def q_read_step(em, st, tmp):
    """Q^T operands of d-step st (both q-blocks) from the query stage: the K
    operand address of the step plus the stage's offset."""
    em(f"v_add_u32 {tmp}, {S_QD}, {KADDR[st]}")
    em.lds_issue(("q", st, 0), f"ds_read_b128 {Q(0, st)}, {tmp} offset:0")
    em.lds_issue(("q", st, 1), f"ds_read_b128 {Q(1, st)}, {tmp} offset:8192")


def q_read(em):
    for st in range(8):
        q_read_step(em, st, AL[0])
    em.lds_drain()


def l_sum(em):
    """l_run of the lane's row over both key halves (lanes l and l ^ 32)."""
    for qb in range(2):
        em(f"v_mov_b32 {ET[qb]}, {LRUN[qb]}")
    em("s_nop 1")
    for qb in range(2):
        em(f"v_permlane32_swap_b32 {LRUN[qb]}, {ET[qb]}")
    for qb in range(2):
        em(f"v_add_f32 {LRUN[qb]}, {LRUN[qb]}, {ET[qb]}")


def output_items(bank, lsum, tmp, zero_o, qnext=False):
    """O^T / l of a unit as bf16 rows, as instruction strings: the output
    descriptor from `bank`, l from the VGPRs lsum (summed over both key
    halves), tmp = 32 VGPR numbers, zero_o: each O^T block zeroed once read,
    by an MFMA of zero operands (the matrix pipe has room beside the
    output's VALU work; 128 AGPR writes would not).  One q-block at a time,
    the rows are staged through the wave's query stage (free then) and
    stored whole, four rows a store, so the first q-block's stores leave
    while the second is converted.  Lane (qc, h) of O[n][qb] register v holds d = 32 n + 8 (v / 4) +
    4 h + v % 4 of row qc of q-block qb: registers 8 half .. 8 half + 7 make
    two 8-byte pieces, of 16-byte chunks 4 n + 2 half and 4 n + 2 half + 1 of
    the lane's row half.  v_permlane32_swap_b32 exchanges vdst's lanes 32-63
    with vsrc's lanes 0-31, so swapping the second piece of the lanes h = 0
    with the first of the lanes h = 1 leaves lane h with chunk 2 st + h
    (st = 2 n + half) whole: written at the K operand address of d-step st
    plus the stage's offset (the stage takes the K tiles' swizzle).  Then
    lane L reads chunk L % 16 of row 4 i + L / 16 (swizzle slot (L % 16) ^
    ((L / 16) << 2) ^ (i % 4), i.e. RL ^ (16 (i % 4)), plus 1024 (i % 4) +
    4096 (i / 4)) and stores it at row 4 i + L / 16: the q-block's rows past
    its row count (the resource size) are dropped; a row without a visible
    key (l = 0) stores zeros.  qnext: the next unit's query rows are copied
    into the stage once it is read."""
    it = ["s_nop 7", "s_nop 7"]  # MFMA results (the last PV) before v_accvgpr_read
    for qb in range(2):
        it.append(f"v_rcp_f32 {AL[qb]}, {lsum[qb]}")
    it += [f"v_cmp_lt_f32_e64 {S_F0}, 0, {lsum[0]}", f"v_cmp_lt_f32_e64 {S_F1}, 0, {lsum[1]}", "s_nop 1",
           f"v_cndmask_b32_e64 {AL[0]}, 0, {AL[0]}, {S_F0}", f"v_cndmask_b32_e64 {AL[1]}, 0, {AL[1]}, {S_F1}"]
    tv = [f"v{x}" for x in tmp[:8]]
    groups = [tmp[8 + 4 * k] for k in range(4)]
    zr = tmp[28]
    if zero_o:
        it += [f"v_mov_b32 v{zr + k}, 0" for k in range(4)]
    for qb, rs_w in ((0, S_RK_W), (1, S_RV_W)):
        for k in range(3):
            it.append(f"v_readlane_b32 {rs_w[k]}, {bank}, {BANK_OB[qb][k]}")
    it += ["s_nop 4", f"s_mov_b32 {S_RK_W[3]}, {RSRC_W3}", f"s_mov_b32 {S_RV_W[3]}, {RSRC_W3}"]
    gi = 0
    for qb in range(2):  # one q-block at a time: its stores leave as early as they can
        if zero_o and qb == 1:  # the first q-block's last rows took the zeros' registers
            it += [f"v_mov_b32 v{zr + k}, 0" for k in range(4)]
        for n in range(4):
            for half in range(2):
                base = 64 + 16 * (2 * n + qb) + 8 * half
                for k in range(8):
                    it.append(f"v_accvgpr_read_b32 {tv[k]}, a{base + k}")
                if zero_o and half == 1:
                    it.append(f"{MF} {O(n, qb)}, v[{zr}:{zr + 3}], v[{zr}:{zr + 3}], 0")
                for k in range(8):
                    it.append(f"v_mul_f32 {tv[k]}, {AL[qb]}, {tv[k]}")
                g = groups[gi % len(groups)]
                gi += 1
                for e in range(4):
                    it.append(f"{CVT} v{g + e}, {tv[2 * e]}, {tv[2 * e + 1]}")
                it.append("s_nop 1")
                it.append(f"v_permlane32_swap_b32 v{g}, v{g + 2}")
                it.append(f"v_permlane32_swap_b32 v{g + 1}, v{g + 3}")
                it.append(f"v_add_u32 {TMPV}, {S_QD}, {KADDR[2 * n + half]}")
                it.append("s_nop 1")
                it.append(f"ds_write_b128 {TMPV}, v[{g}:{g + 3}] offset:{8192 * qb}")
        it.append("s_waitcnt lgkmcnt(0)")
        # whole rows back, four a store
        rsrc = S_RK if qb == 0 else S_RV
        for i in range(8):
            y = tmp[4 * i]
            if i % 4:
                it.append(f"v_xor_b32 {TMPV}, {16 * (i % 4)}, {RL}")
                addr = TMPV
            else:
                addr = RL
            it.append(f"ds_read_b128 v[{y}:{y + 3}], {addr} offset:{8192 * qb + 4096 * (i // 4) + 1024 * (i % 4)}")
        it.append("s_waitcnt lgkmcnt(0)")
        for i in range(8):
            y = tmp[4 * i]
            it.append(f"s_mul_i32 {S_TMP}, {S_O4}, {i}")
            it.append(f"buffer_store_dwordx4 v[{y}:{y + 3}], {OOFF}, {rsrc}, {S_TMP} offen")
        it.append("s_nop 1")
    if qnext:
        # the next unit's query rows into the stage (none when it has no tile)
        pre = Items()
        q_prefetch(pre, BANKN, guard=True)
        it += pre
    return it


def zero_output(em, bank):
    """A unit whose rows see no key: zeros for its rows (row 4 i + L / 16,
    chunk L % 16 from lane L, i = 0..7)."""
    for qb, rs_w in ((0, S_RK_W), (1, S_RV_W)):
        for k in range(3):
            em(f"v_readlane_b32 {rs_w[k]}, {bank}, {BANK_OB[qb][k]}")
    em("s_nop 4")
    em(f"s_mov_b32 {S_RK_W[3]}, {RSRC_W3}")
    em(f"s_mov_b32 {S_RV_W[3]}, {RSRC_W3}")
    for k in range(4):
        em(f"v_mov_b32 v{k}, 0")
    for rs in (S_RK, S_RV):
        for i in range(8):
            em(f"s_mul_i32 {S_TMP}, {S_O4}, {i}")
            em(f"buffer_store_dwordx4 v[0:3], {OOFF}, {rs}, {S_TMP} offen")


def unit_init(em, paged):
    """Per-unit loop state: running max and sum, tile count, block ids and
    cache rows of tiles 0 and 1."""
    em(f"v_mov_b32 {MRUN[0]}, 0xff800000")
    em(f"v_mov_b32 {MRUN[1]}, 0xff800000")
    em(f"v_mov_b32 {LRUN[0]}, 0")
    em(f"v_mov_b32 {LRUN[1]}, 0")
    em(f"s_sub_u32 {S_LAST}, {S_NT}, 1")
    em(f"s_mov_b32 {S_J}, 0")
    if paged:
        em(f"s_mov_b32 {S_KOFF}, 0")
        em(f"s_mov_b32 {S_LB}, 0")
        for t in range(2):
            em(f"s_mov_b32 {S_B[t]}, {S_BLK012[t]}")
            block_row(em, S_ROW[t], S_B[t])
            advance_tile(em)
    else:
        em(f"s_mov_b32 {S_ROW[0]}, 0")
        em(f"s_mov_b32 {S_ROW[1]}, 64")


def unit_start(em, lbl, qnext=True):
    """The next unit's query rows into the stage (the current unit's are in
    the Q^T registers), the plan record of the unit after it (S_U2), the
    claim of the one after that, and whether the current unit chains into
    the next (two tiles or more here, a tile there)."""
    if qnext:
        em(f"s_cmp_eq_u32 {S_NNT}, 0")
        em(f"s_cbranch_scc1 {lbl}noq")
        q_prefetch(em, BANKN)
        em(f"{lbl}noq:")
    emit_items(em, record_load_items(S_U2))
    claim(em, lbl)
    em(f"s_cmp_gt_u32 {S_NT}, 1")
    em(f"s_cselect_b32 {S_FLAGS}, 1, 0")
    em(f"s_cmp_eq_u32 {S_NNT}, 0")
    em(f"s_cselect_b32 {S_FLAGS}, 0, {S_FLAGS}")


def block_iteration(em, paged, par, kind, lbl):
    """Iteration j (parity par) of one of these kinds:
      fresh0  a unit's first tile after a fresh start (no PV),
      chain0  a unit's first tile in a chain: the PV of the previous unit's
              last tile (V and P of parity 1 - par) and its output beside
              this unit's QK^T of tile 1,
      main    a tile between,
      last    a unit's last tile ending the pipeline: no K fill, no QK^T,
      lastc   a unit's last tile chaining into the next: the next unit's
              Q^T read and QK^T of its tile 0.
    Fills: K tile j+2 (or the next unit's tile 0 / 1) and V tile j+1 (or
    the next unit's tile 0; none in a last iteration), spread over segment
    A.  Paged: the block id of tile j+2 (from the record for a first tile,
    else loaded an iteration earlier) is taken and the load of tile j+3's
    issued.  Iterations after the first read the claim slot and load the
    claimed unit's plan record.  V operand reads: segment A's PV reads
    operands AHEAD.. (the iteration before read the first AHEAD), the VADDR
    registers then move to this iteration's V buffer and segment B reads
    the first AHEAD operands of the PV of tile j, behind its QK^T's K
    operand reads."""
    first = kind in ("fresh0", "chain0")
    pv = kind != "fresh0"
    qk = kind != "last"
    ppar, spar = 1 - par, 1 - par
    em.lds = early_tags() if pv else []
    if kind == "lastc":  # the next unit's query rows, copied at the unit's start
        em("s_waitcnt vmcnt(0)")
    mark(em, 0)
    if kind == "lastc":
        vfill = fill_tile(paged, "v", None, None, None, None, nxt="v0")
    elif kind != "last":
        vfill = fill_tile(paged, "v", S_ROW[1], S_J, S_B[1] if paged else None, None, tile_add=1)
    else:
        vfill = []
    fill = vfill if V_FILL_FIRST else []
    fill += tile_rows_items(paged, first)
    fill += [] if kind == "last" else fill_tile(paged, "k", S_ROW[2], S_T[2], S_B[2] if paged else None, par,
                                               nxt="one" if kind == "lastc" else "sel")
    if not V_FILL_FIRST:
        fill += vfill
    # ---- segment A
    pairs = exp_pairs(par)
    touched = set()
    a_items = (row_max(par) + max_update(True)) if first else []
    a_items += exp_items(pairs[:NA], 0, touched)
    b_items = exp_items(pairs[NA:], NA, touched) + tile_sum_items()
    assert len(touched) == 6, "every partial row sum is written each tile"
    if kind == "lastc":  # the unit after next decoded, the units moved on
        dec = Items()
        decode(dec, S_U2, paged)
        advance_units(dec)
        b_items += dec
    if kind == "chain0":  # the previous unit's output first: its stores leave early
        pt = 128 + 32 * ppar  # the previous P, read by segment A's PV, is free in segment B
        b_items = output_items(BANKP, LPREV, list(range(pt, pt + 32)), zero_o=True, qnext=True) + b_items
    if not pv:
        emit_items(em, fill)
        emit_items(em, a_items)
        emit_items(em, v_rotate_items())
        mark(em, 1)
        for i in range(AHEAD):
            k_read(em, spar, i)
    else:
        lead = 0  # VALU work before the first MFMA (none: measured fastest of 0, 2, 4, 6, 8, 12)
        emit_items(em, a_items[:lead])
        # the fill's scalar setup and loads share the first FILL_SLOTS slots
        slots = spread(a_items[lead:], 32)
        fs = spread(fill, FILL_SLOTS)
        for k in range(FILL_SLOTS):
            slots[k] = fs[k] + slots[k]
        # the VADDR move after the last V read (at step 15 - AHEAD)
        rot = v_rotate_items()
        slots[24] = [rot[0]] + slots[24]
        for k, x in enumerate(rot[1:]):
            slots[25 + k % 7] = [x] + slots[25 + k % 7]
        for i in range(16):
            em.lds_wait(("v", i, 1))
            mf = pv_mfmas(em, i, ppar)
            em(mf[0])
            read_ahead_a(em, spar, i, not qk)
            if kind == "lastc" and 1 <= i <= 8:
                q_read_step(em, i - 1, AL[0])
            emit_items(em, slots[2 * i])
            em(mf[1])
            emit_items(em, slots[2 * i + 1])
        mark(em, 1)
    # ---- segment B
    slots = spread(b_items, 32)
    for i in range(16 if qk else 0):
        em.lds_wait(("k", i))
        mf = qk_mfmas(i, spar)
        em(mf[0])
        if i + AHEAD < 16:
            k_read(em, spar, i + AHEAD)
        else:  # the next PV's first operands, from this iteration's V buffer
            v_read(em, i + AHEAD - 16)
        emit_items(em, slots[2 * i])
        em(mf[1])
        emit_items(em, slots[2 * i + 1])
    if not qk:
        for i in range(AHEAD):
            v_read(em, i)
        emit_items(em, b_items)
    # The tile's row sums, taken with the running max of the tiles before:
    # past SUM_LIMIT or not finite (a max that was stale or still -inf) on
    # any lane, the slow path redoes the tile with its own max.
    em(f"v_add_f32 {ET[0]}, {SW[0]}, {SW[1]}")
    em(f"v_cmp_nge_f32 vcc, {SUM_LIMIT}, {ET[0]}")
    em(f"s_or_b64 vcc, vcc, {S_MINF}")
    em(f"s_cbranch_scc1 {lbl}_slow")
    for qb in range(2):
        em(f"v_add_f32 {LRUN[qb]}, {LRUN[qb]}, {SW[qb]}")
    em(f"{lbl}_summed:")
    mark(em, 2)
    # ---- next tile's mask limit, rotation, barrier
    em(f"v_subrev_u32 {LIM[0]}, 64, {LIM[0]}")
    em(f"v_subrev_u32 {LIM[1]}, 64, {LIM[1]}")
    if paged:
        em(f"s_mov_b32 {S_B[0]}, {S_B[1]}")
        em(f"s_mov_b32 {S_B[1]}, {S_B[2]}")
    em(f"s_mov_b32 {S_ROW[0]}, {S_ROW[1]}")
    em(f"s_mov_b32 {S_ROW[1]}, {S_ROW[2]}")
    vb_advance(em)
    # chain0's output stores and the next unit's query-row copies (its last
    # 32 vector memory operations) may drain
    em(f"s_waitcnt vmcnt({32 if kind == 'chain0' else 0})")
    mark(em, 3)
    if first:
        claim_publish(em, lbl)
    em("s_barrier")
    mark(em, 4)


def block_slow(em, par, lbl):
    """Slow path of tile j (parity par), out of line: the running max moves
    to the tile's max, l_run and (where alpha != 1 on some lane) O scale by
    alpha, and P_j and the tile's row sums are redone with the new max.  The
    PV MFMAs that wrote O were issued a segment earlier; 16 wait states
    cover an MFMA result before v_accvgpr_read regardless."""
    em(f"{lbl}_slow:")
    emit_items(em, row_max(par))
    emit_items(em, max_update(False))
    em(f"v_cmp_neq_f32_e64 {S_F0}, 1.0, {AL[0]}")
    em(f"v_cmp_neq_f32_e64 {S_F1}, 1.0, {AL[1]}")
    em(f"s_or_b64 {S_F0}, {S_F0}, {S_F1}")
    em(f"s_cbranch_scc0 {lbl}_scaled")
    em("s_nop 7")
    em("s_nop 7")
    for r in range(16):
        regs = [64 + 8 * r + k for k in range(8)]
        for k, a in enumerate(regs):
            em(f"v_accvgpr_read_b32 {ET[k]}, a{a}")
        for k, a in enumerate(regs):
            qb = ((a - 64) // 16) % 2
            em(f"v_mul_f32 {ET[k]}, {ET[k]}, {AL[qb]}")
        for k, a in enumerate(regs):
            em(f"v_accvgpr_write_b32 a{a}, {ET[k]}")
    em(f"{lbl}_scaled:")
    touched = set()
    emit_items(em, exp_items(exp_pairs(par), 0, touched))
    emit_items(em, tile_sum_items())
    for qb in range(2):
        em(f"v_add_f32 {LRUN[qb]}, {LRUN[qb]}, {SW[qb]}")
    em(f"s_branch {lbl}_summed")


def block_mask(em, par):
    """-inf on the scores of S_j past each row's last visible key: register v
    of S[kb][qb] holds key 32 kb + 8 (v / 4) + v % 4 + 4 h of the tile, and
    LIM[qb] = the lane's last visible key - 4 h.  Compares write four lane
    masks in turn, so each v_cndmask reads a mask written four instructions
    earlier (a VALU-written mask needs two wait states before a VALU reads it)."""
    masks = [S_F0, S_F1, S_NEED[0], S_NEED[1]]
    cells = [(qb, kb, v) for qb in range(2) for kb in range(2) for v in range(16)]
    for g0 in range(0, len(cells), 4):
        grp = cells[g0:g0 + 4]
        for k, (qb, kb, v) in enumerate(grp):
            c = 32 * kb + 8 * (v // 4) + (v % 4)
            em(f"v_cmp_gt_i32_e64 {masks[k]}, {c}, {LIM[qb]}")
        for k, (qb, kb, v) in enumerate(grp):
            em(f"v_cndmask_b32_e64 {Sr(par, kb, qb, v)}, {Sr(par, kb, qb, v)}, {NINF}, {masks[k]}")


def block_prologue(em):
    """QK^T of a fresh unit's tile 0 (K_0 in K buffer 0, Q^T in its
    registers), O^T zeroed beside it, four AGPR writes a MFMA."""
    em("s_nop 1")
    for i in range(AHEAD):
        k_read(em, 0, i)
    zero = [f"v_accvgpr_write_b32 a{64 + r}, 0" for r in range(128)]
    for i in range(16):
        em.lds_wait(("k", i))
        for x in qk_mfmas(i, 0):
            em(x)
            for _ in range(4):
                em(zero.pop(0))
        if i + AHEAD < 16:
            k_read(em, 0, i + AHEAD)
    assert not zero
    # every wave has read K_0 before iteration 0 refills its buffer
    em("s_waitcnt lgkmcnt(0)")
    em.lds = []
    em("s_barrier")
    mark(em, 5)
    em("s_nop 7")
    em("s_nop 4")


def block_pv_only(em, par):
    """PV of the last tile (P of parity par): its first AHEAD V operands
    were read by the last iteration."""
    for i in range(16):
        em.lds_wait(("v", i, 1))
        for x in pv_mfmas(em, i, par):
            em(x)
        if i + AHEAD < 16:
            v_read(em, i + AHEAD)
    em.lds_drain()


def claim_slot_read(em):
    """S_U2 <- the unit the current one claimed at its start (its first
    iteration published it; every wave has passed a barrier since)."""
    slot_address(em, TMPV)
    em(f"ds_read_b32 {AL[1]}, {TMPV}")
    em("s_waitcnt lgkmcnt(0)")
    em(f"v_readfirstlane_b32 {S_U2}, {AL[1]}")
    em("s_nop 1")
    em(f"s_lshl_b32 {S_U2}, {S_U2}, 3")
    em(f"s_add_u32 {S_U2}, {S_U2}, {S_XCD}")


def program(paged):
    em = Emitter()
    u = "L%=_"
    mark(em, None)
    em("s_nop 4")
    em(f"v_mov_b32 {NINF}, 0xff800000")
    em(f"s_mov_b32 {S_IT}, 0")
    em(f"s_mov_b32 {S_VB}, 0")
    # ---- the work-group's first three units (claimed by the caller): the
    # first two decoded, the third's record loaded by the first's start
    emit_items(em, record_load_items(S_U0))
    em("s_waitcnt vmcnt(0)")
    decode(em, S_U0, paged)
    em(f"v_mov_b32 {BANKN}, {BANKN2}")
    emit_items(em, record_load_items(S_U1))
    em("s_waitcnt vmcnt(0)")
    decode(em, S_U1, paged)
    advance_units(em)
    set_lim(em)
    em(f"s_mov_b32 {S_U2}, {S_U2IN}")
    em(f"s_cmp_eq_u32 {S_NT}, 0")
    em(f"s_cbranch_scc1 {u}s0")
    q_prefetch(em, BANKU)
    cur = []
    for tl, (lo, hi, rec) in enumerate(BANK_NK):
        regs = DT[12 + 3 * tl: 15 + 3 * tl]  # not the fill resources k_prefetch writes
        cur.append(tuple(regs))
        readlanes(em, [(regs[0], BANKU, lo), (regs[1], BANKU, hi), (regs[2], BANKU, rec)])
    k_prefetch(em, cur, BANKU)
    em(f"{u}s0:")
    em("s_waitcnt vmcnt(0)")
    em("s_barrier")
    em(f"s_cmp_eq_u32 {S_NT}, 0")
    em(f"s_cbranch_scc1 {u}fresh")
    q_read(em)
    # ---- a unit from a fresh start: K_0, K_1 in K buffers 0, 1, Q^T read
    em(f"{u}fresh:")
    em(f"s_cmp_eq_u32 {S_NT}, 0")
    em(f"s_cbranch_scc1 {u}zero")
    unit_init(em, paged)
    unit_start(em, f"{u}f")
    block_prologue(em)
    em(f"s_cmp_gt_i32 {S_JM}, 0")
    em(f"s_cbranch_scc1 {u}i0nomask")
    block_mask(em, 0)
    em(f"{u}i0nomask:")
    block_iteration(em, paged, 0, "fresh0", f"{u}i0")
    em(f"s_mov_b32 {S_J}, 1")
    em(f"s_branch {u}top")
    # ---- a unit in a chain, its first iteration at parity p
    for p in (0, 1):
        em(f"{u}chain{p}:")
        unit_init(em, paged)
        unit_start(em, f"{u}c{p}", qnext=False)
        em(f"s_cmp_gt_i32 {S_JM}, 0")
        em(f"s_cbranch_scc1 {u}c{p}nomask")
        block_mask(em, p)
        em(f"{u}c{p}nomask:")
        block_iteration(em, paged, p, "chain0", f"{u}c{p}i")
        em(f"s_mov_b32 {S_J}, 1")
        em(f"s_branch {u}{'top' if p == 0 else 'mid'}")
    # ---- iterations 1, 2, ... (parity 1 at top, 0 at mid)
    em(f"{u}top:")
    for par in (1, 0):
        if par == 0:
            em(f"{u}mid:")
        em(f"s_cmp_gt_i32 {S_J}, {S_LAST}")
        em(f"s_cbranch_scc1 {u}drain{1 - par}")
        em(f"s_cmp_lt_i32 {S_J}, {S_JM}")
        em(f"s_cbranch_scc1 {u}nomask{par}")
        block_mask(em, par)
        em(f"{u}nomask{par}:")
        em(f"s_cmp_eq_u32 {S_J}, {S_LAST}")
        em(f"s_cbranch_scc1 {u}last{par}")
        block_iteration(em, paged, par, "main", f"{u}m{par}")
        em(f"s_add_u32 {S_J}, {S_J}, 1")
    em(f"s_branch {u}top")
    # ---- a unit's last iteration (j = S_LAST >= 1), out of line
    for par in (1, 0):
        em(f"{u}last{par}:")
        em(f"s_bitcmp1_b32 {S_FLAGS}, 0")
        em(f"s_cbranch_scc1 {u}lastc{par}")
        block_iteration(em, paged, par, "last", f"{u}l{par}")
        em(f"s_branch {u}drain{par}")
        em(f"{u}lastc{par}:")
        block_iteration(em, paged, par, "lastc", f"{u}lc{par}")
        em(f"s_branch {u}trans{par}")
    # ---- out-of-line slow paths
    block_slow(em, 0, f"{u}i0")
    for p in (0, 1):
        block_slow(em, p, f"{u}c{p}i")
    for par in (1, 0):
        block_slow(em, par, f"{u}m{par}")
        block_slow(em, par, f"{u}l{par}")
        block_slow(em, par, f"{u}lc{par}")
    # ---- the pipeline ends after a last iteration at parity par: the next
    # unit's first key tiles and query rows, the last PV, the output
    for par in (0, 1):
        em(f"{u}drain{par}:")
        em("s_waitcnt vmcnt(0) lgkmcnt(0)")
        em.lds = []
        em(f"s_cmp_eq_u32 {S_NNT}, 0")
        em(f"s_cbranch_scc1 {u}d{par}nonext")
        k_prefetch(em, [(lo, hi, rec) for (lo, hi), rec in zip(S_NK, S_NREC)], BANKN)
        q_read(em)
        em(f"{u}d{par}nonext:")
        block_pv_only(em, par)
        l_sum(em)
        emit_items(em, output_items(BANKU, LRUN, list(range(32)), zero_o=False))
        em(f"s_branch {u}next")
    # ---- a unit's last iteration chained into the next (its QK^T_0 done,
    # the units moved on beside it)
    for par in (0, 1):
        em(f"{u}trans{par}:")
        l_sum(em)
        em(f"v_mov_b32 {LPREV[0]}, {LRUN[0]}")
        em(f"v_mov_b32 {LPREV[1]}, {LRUN[1]}")
        set_lim(em)
        claim_slot_read(em)
        em(f"s_add_u32 {S_IT}, {S_IT}, 1")
        em(f"s_branch {u}chain{1 - par}")
    # ---- a unit whose rows see no key (the pipeline is empty)
    em(f"{u}zero:")
    unit_start(em, f"{u}z")
    em("s_waitcnt vmcnt(0)")
    claim_publish(em, f"{u}z")
    em("s_barrier")
    em(f"s_cmp_eq_u32 {S_NNT}, 0")
    em(f"s_cbranch_scc1 {u}znonext")
    k_prefetch(em, [(lo, hi, rec) for (lo, hi), rec in zip(S_NK, S_NREC)], BANKN)
    q_read(em)
    em(f"{u}znonext:")
    zero_output(em, BANKU)
    # ---- after an ended pipeline: the next unit, if any, from a fresh start
    # (its first key tiles and the record landed: the output's 16 stores
    # were issued last)
    em(f"{u}next:")
    em(f"s_cmp_eq_u32 {S_NEX}, 0")
    em(f"s_cbranch_scc1 {u}exit")
    em("s_waitcnt vmcnt(16)")
    decode(em, S_U2, paged)
    advance_units(em)
    set_lim(em)
    claim_slot_read(em)
    em(f"s_add_u32 {S_IT}, {S_IT}, 1")
    em("s_barrier")
    em(f"s_branch {u}fresh")
    em(f"{u}exit:")
    mark(em, 6)
    em("s_waitcnt vmcnt(0) lgkmcnt(0)")
    em("s_nop 7")
    em("s_nop 7")
    em("s_nop 3")
    return em.lines


# Everything the statement writes except what it restores (exec): the
# inputs it reads are left as they came.
INPUT_REGS = set()  # filled from the C++ operand list by the checker
CLOBBERS = (
    [f"v{i}" for i in range(0, 192)] + [f"v{i}" for i in range(216, 246)] + [f"v{i}" for i in range(249, 253)]
    + [f"a{i}" for i in range(0, 256)]
    + [f"s{i}" for i in range(24, 32)] + [f"s{i}" for i in range(34, 37)] + ["s38", "s39"]
    + [f"s{i}" for i in range(40, 54)] + [f"s{i}" for i in range(56, 60)] + [f"s{i}" for i in range(64, 101)]
    + ["vcc", "scc", "m0", "memory"]
)


def render(name, lines):
    out = [f"#define {name} \\"]
    for ln in lines:
        out.append(f'  "{ln}\\n" \\')
    out.append('  ""')
    return "\n".join(out)


def main():
    here = os.path.dirname(os.path.abspath(__file__))
    paged = program(True)
    local = program(False)
    set_element(True)
    paged16 = program(True)
    local16 = program(False)
    set_element(False)
    clob = ", ".join(f'"{c}"' for c in CLOBBERS)
    text = [
        "// Generated by gen_prefill_mx.py; do not edit by hand.",
        "// The persistent loop of the MFMA prefill kernel (see paged_prefill_mx.hip).",
        "#pragma once",
        "",
        render("NVS_PREFILL_MX_ASM_PAGED", paged),
        "",
        render("NVS_PREFILL_MX_ASM_LOCAL", local),
        "",
        render("NVS_PREFILL_MX_ASM_PAGED_F16", paged16),
        "",
        render("NVS_PREFILL_MX_ASM_LOCAL_F16", local16),
        "",
        f"#define NVS_PREFILL_MX_CLOBBERS {clob}",
        "",
    ]
    path = os.path.join(here, "prefill_mx_asm.inc")
    with open(path, "w") as f:
        f.write("\n".join(text))
    print(f"wrote {path}: {len(paged)} + {len(local)} lines (and as many for fp16)", file=sys.stderr)


if __name__ == "__main__":
    main()
