#!/usr/bin/env python3
"""Generator of the hand-scheduled tile loop of the MFMA prefill kernel
(paged_prefill_mx.hip) for gfx950.

Writes prefill_mx_asm.inc next to this file: two string-literal macros
(NVS_PREFILL_MX_ASM_PAGED, NVS_PREFILL_MX_ASM_LOCAL), each the body of one
inline-asm statement that runs a work item's whole tile loop.  Run it after
editing this file:  python nanovllm_self_amd/csrc/gen_prefill_mx.py

Per wave: 64 query rows as two 32-row q-blocks (qb), one 64-key tile per
iteration, v_mfma_f32_32x32x16_bf16 throughout:
  S^T[kb][qb] (32 keys x 32 q)  = K . Q^T   16 d-steps x ... = 32 MFMAs
  O^T[n][qb]  (32 d x 32 q)    += V^T . P^T                   32 MFMAs
Iteration j: segment A runs PV of tile j-1 beside the row max / running-max
update of S_j and the first exponentials; segment B runs QK of tile j+1
beside the rest of S_j's exponentials, the bf16 packing of P_j and the row
sums.  K/V operands are read from LDS into an AGPR ring four operands ahead
of their MFMAs; the next tiles are copied HBM -> LDS with buffer loads that
write LDS directly (out-of-range rows read as zero).

Register map (fixed; the C++ side binds inputs and outputs to it):
  v[0:127]    S_j / S_{j+1}: S[par][kb][qb] = v[64 par + 16 (2 kb + qb) ..]
  v[128:191]  P_j / P_{j-1}: P[par][qb][m] = v[128 + 32 par + 16 qb + 4 m ..]
  v[192:199]  K operand LDS addresses, one per d-step st (K buffer 0, kb 0)
  v[200:207]  V operand LDS addresses, per (d-block n, key half e)
  v[208:211]  K DMA lane offsets, v[212:215] V DMA lane offsets
  v216-217 m_run, v218-219 l_run (out), v220-221 mask limit (in/out)
  v222 -inf, v223 bf16 (1, 1), v224-231 softmax temporaries,
  v232-239 exponential temporaries, v240 block id
  v244-v248   output descriptor (in), v[0:31] output temporaries
  a[0:63]     Q^T operands: Q[qb][st] = a[32 qb + 4 st ..]   (in)
  a[64:191]   O^T accumulators: O[n][qb] = a[64 + 16 (2 n + qb) ..]
  a[192:223]  V operand ring (8 slots), a[224:255] K operand ring (8 slots)
  s[33:63]    scalar inputs, s[64:99] loop state
After the loop the statement copies the next unit's key tiles 0 and 1 into
the K buffers (both free then), runs the last PV, normalises O and stores it
as bf16 rows straight from registers: v_permlane32_swap_b32 pairs the two
lane halves' 8-byte pieces into 16-byte chunks of one row each.
"""
from __future__ import annotations

import os
import sys

MF = "v_mfma_f32_32x32x16_bf16"

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
DMAK = [f"v{208 + i}" for i in range(4)]
DMAV = [f"v{212 + i}" for i in range(4)]
MRUN = ["v216", "v217"]
LRUN = ["v218", "v219"]
LIM = ["v220", "v221"]
NINF = "v222"
ONES = "v223"
MX = ["v224", "v225"]
SW = ["v226", "v227"]
NMS = ["v228", "v229"]
AL = ["v230", "v231"]
ET = [f"v{232 + i}" for i in range(8)]
BLKV = "v240"
X3 = ["v241", "v242"]  # third partial row sum

# scalar inputs
S_KBASE, S_VBASE = "s[40:41]", "s[42:43]"
S_KBASE_LO, S_KBASE_HI, S_VBASE_LO, S_VBASE_HI = "s40", "s41", "s42", "s43"
S_KROW, S_VROW, S_K, S_NT, S_JM, S_BS, S_NB, S_M0W, S_SCALE = (
    "s44", "s45", "s46", "s47", "s48", "s49", "s50", "s51", "s52")
S_RBT = "s[36:39]"  # buffer resource of the sequence's block-table row (paged)
S_RBT_NREC = "s38"  # its size in bytes: 4 x the blocks of the sequence
S_BLK012 = ["s33", "s34", "s35"]  # block ids of tiles 0, 1, 2 (paged; from the plan)
S_WID = "s53"        # the wave's index in the work-group
S_CNT = "s[54:55]"   # address of the XCD's unit counter
CLAIM = "v243"       # out: the claimed counter value (wave 0, lane 0)
# The unit's output and the next unit's first key tiles, handled after the loop:
OD = ["v244", "v245", "v246", "v247"]  # output of q-block 0: base lo, base hi; bytes of q-block 0, 1
OOFF = "v248"        # lane offset of the output rows: (lane % 32) x row stride + 16 (lane / 32)
S_NK = [("s56", "s57"), ("s58", "s59")]  # next unit's key tiles 0, 1: first byte (lo, hi)
S_NREC = ["s60", "s61"]  # their bytes (rows x key row stride; 0 reads nothing)
S_FLAGS = "s62"      # bit 0: prefetch the next unit's key tiles 0 and 1
S_ODELTA = "s63"     # q-block 1's output base minus q-block 0's, in bytes
# loop state
S_J, S_LAST = "s64", "s65"
S_B = ["s66", "s67", "s68"]        # block ids of tiles j, j+1, j+2 (paged)
S_ROW = ["s69", "s70", "s71"]      # first cache row of tiles j, j+1, j+2
S_KOFF, S_LB = "s72", "s73"        # key offset in block / logical block of the next block-id read
S_RK, S_RV = "s[76:79]", "s[80:83]"  # buffer resources of the K and V fills
S_RK_W = ["s76", "s77", "s78", "s79"]
S_RV_W = ["s80", "s81", "s82", "s83"]
S_F0, S_F1 = "s[84:85]", "s[86:87]"
S_NEED = ["s[94:95]", "s[96:97]"]  # per q-block lane masks (temporaries)
S_MINF = "s[98:99]"  # lanes whose running max is still -inf (no visible key yet)
S_T = ["s88", "s89", "s90", "s91"]
S_BOK = "s93"  # 1 if the block-id load in flight is of a block of the sequence

LDS_V0 = 32768      # V buffer 0 (K buffers at 0 and 16384)
TILE = 16384        # bytes of one 64-key bf16 tile
RSRC_W3 = "0x20000"  # raw buffer: 32-bit data format, no swizzle, no stride


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
        """Wait until the LDS op `tag` has completed (LDS returns in order)."""
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
# no exponential of a tile exceeds 2^16 times the row's running max term
SUM_LIMIT = "0x47800000"  # 65536.0


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
            it.append(f"v_cvt_pk_bf16_f32 {p}, {t[k][0]}, {t[k][1]}")
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
def v_read(em, par_buf, i):
    """V operand i (m = i // 4, n = i % 4) of the V buffer par_buf into ring slot i % 8."""
    m, n = divmod(i, 4)
    _, lo, hi = VSLOT(i % 8)
    off = TILE * par_buf + 4096 * m
    em.lds_issue(("v", i, 0), f"ds_read_b64_tr_b16 {lo}, {VADDR[(n, 0)]} offset:{off}")
    em.lds_issue(("v", i, 1), f"ds_read_b64_tr_b16 {hi}, {VADDR[(n, 1)]} offset:{off}")


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
READ_EARLY = True  # issue each read-ahead right after the slot's first MFMA
V_FIRST = True  # issue segment A's first V reads before the fills' set-up
NA = 12  # exponential pairs of segment A


def read_ahead_a(em, ppar, spar, i, last=False):
    """Segment A's read-ahead after PV operand i: V operand i + AHEAD, or,
    in the last AHEAD slots, the first K operands of segment B (none in a
    unit's last iteration, whose segment B has no QK^T)."""
    if i + AHEAD < 16:
        v_read(em, ppar, i + AHEAD)
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
def fill_tile(paged, which, row, tile, blk, par_dst):
    """Instructions that copy one 64-key tile (K or V) into buffer par_dst:
    row = first cache row of the tile (SGPR), tile = SGPR holding its index
    (for the row count), blk = its block id (paged; < 0: missing).  Returns
    a list whose items are instruction strings or groups (lists) that must
    stay together: each m0 write, its wait state and its direct-to-LDS load."""
    base_lo, base_hi = (S_KBASE_LO, S_KBASE_HI) if which == "k" else (S_VBASE_LO, S_VBASE_HI)
    rowb = S_KROW if which == "k" else S_VROW
    rs = S_RK_W if which == "k" else S_RV_W
    rsrc = S_RK if which == "k" else S_RV
    offs = DMAK if which == "k" else DMAV
    t0 = S_T[0] if which == "k" else S_T[1]
    out = [
        f"s_mul_i32 {rs[0]}, {row}, {rowb}",
        f"s_mul_hi_u32 {rs[1]}, {row}, {rowb}",
        f"s_add_u32 {rs[0]}, {rs[0]}, {base_lo}",
        f"s_addc_u32 {rs[1]}, {rs[1]}, {base_hi}",
        f"s_and_b32 {rs[1]}, {rs[1]}, 0xffff",
        # rows of the tile that hold keys: clamp(K - 64 t, 0, 64)
        f"s_lshl_b32 {t0}, {tile}, 6",
        f"s_sub_i32 {t0}, {S_K}, {t0}",
        f"s_max_i32 {t0}, {t0}, 0",
        f"s_min_i32 {t0}, {t0}, 64",
        f"s_mul_i32 {rs[2]}, {t0}, {rowb}",
    ]
    if paged:
        out += [f"s_cmp_lt_i32 {blk}, 0", f"s_cselect_b32 {rs[2]}, 0, {rs[2]}"]
    out.append(f"s_mov_b32 {rs[3]}, {RSRC_W3}")
    dst = (0 if which == "k" else LDS_V0) + TILE * par_dst
    for i in range(4):
        out.append([f"s_add_u32 m0, {S_M0W}, {dst + 1024 * i}", "s_nop 0",
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


def issue_block_id(em):
    """Vector load of the block id of logical block S_LB into BLKV (every
    lane the same address); S_BOK records whether S_LB is a block of the
    sequence.  The loop's vmcnt(0) before each barrier completes it."""
    em(f"s_lshl_b32 {S_T[2]}, {S_LB}, 2")
    em(f"v_mov_b32 {ET[0]}, {S_T[2]}")
    em(f"buffer_load_dword {BLKV}, {ET[0]}, {S_RBT}, 0 offen")
    em(f"s_cmp_lt_u32 {S_T[2]}, {S_RBT_NREC}")
    em(f"s_cselect_b32 {S_BOK}, 1, 0")


def take_block_id(em, dst):
    """dst <- the block id loaded by issue_block_id, or -1 where the
    logical block is past the sequence's or the id is outside the pool."""
    em(f"v_readfirstlane_b32 {dst}, {BLKV}")
    em("s_nop 0")
    em(f"s_cmp_lt_u32 {dst}, {S_NB}")
    em(f"s_cselect_b32 {dst}, {dst}, -1")
    em(f"s_cmp_eq_u32 {S_BOK}, 0")
    em(f"s_cselect_b32 {dst}, -1, {dst}")


# ----------------------------------------------------------------- blocks
def block_iteration(em, paged, par, first, lbl, last=False):
    """Iteration j (parity par): fill K_{j+2}, V_j (spread over segment A);
    segment A (PV_{j-1} unless first) beside the max / m update and the
    first exponentials; segment B (QK_{j+1}) beside the rest; the row-sum
    check; barrier.  Paged: the block id of tile j+2 (loaded an iteration
    earlier; iteration 0: from the plan) is taken first and the load of
    tile j+3's issued.  The unit's last iteration (last) has no tile j+1:
    no K fill, no K reads and segment B is its VALU work alone."""
    ppar, spar = 1 - par, 1 - par
    if V_FIRST and not first:
        for i in range(AHEAD):
            v_read(em, ppar, i)
    # ---- tile rows of the fills
    if paged:
        if first:
            em(f"s_mov_b32 {S_B[2]}, {S_BLK012[2]}")
        else:
            take_block_id(em, S_B[2])
        block_row(em, S_ROW[2], S_B[2])
        advance_tile(em)
        issue_block_id(em)  # tile j+3, taken at iteration j+1
    else:
        em(f"s_add_u32 {S_T[2]}, {S_J}, 2")
        em(f"s_lshl_b32 {S_ROW[2]}, {S_T[2]}, 6")
    em(f"s_add_u32 {S_T[2]}, {S_J}, 2")
    mark(em, 0)
    fill = [] if last else fill_tile(paged, "k", S_ROW[2], S_T[2], S_B[2] if paged else None, par)
    fill += fill_tile(paged, "v", S_ROW[0], S_J, S_B[0] if paged else None, par)
    # ---- segment A
    pairs = exp_pairs(par)
    na = NA  # exponential pairs in segment A (a multiple of 4)
    touched = set()
    a_items = (row_max(par) + max_update(True)) if first else []
    a_items += exp_items(pairs[:na], 0, touched)
    b_items = exp_items(pairs[na:], na, touched) + tile_sum_items()
    assert len(touched) == 6, "every partial row sum is written each tile"
    if first:
        emit_items(em, fill)
        emit_items(em, a_items)
        mark(em, 1)
        for i in range(AHEAD):
            k_read(em, spar, i)
    else:
        if not V_FIRST:
            for i in range(AHEAD):
                v_read(em, ppar, i)
        lead = 8  # VALU work before the first MFMA waits for its operand
        emit_items(em, a_items[:lead])
        # the fill's scalar setup and loads share the first 16 slots
        slots = spread(a_items[lead:], 32)
        fs = spread(fill, 16)
        for k in range(16):
            slots[k] = fs[k] + slots[k]
        for i in range(16):
            em.lds_wait(("v", i, 1))
            mf = pv_mfmas(em, i, ppar)
            em(mf[0])
            if READ_EARLY:
                read_ahead_a(em, ppar, spar, i, last)
            emit_items(em, slots[2 * i])
            em(mf[1])
            emit_items(em, slots[2 * i + 1])
            if not READ_EARLY:
                read_ahead_a(em, ppar, spar, i, last)
        mark(em, 1)
    # ---- segment B
    slots = spread(b_items, 32)
    for i in range(0 if last else 16):
        em.lds_wait(("k", i))
        mf = qk_mfmas(i, spar)
        em(mf[0])
        if READ_EARLY and i + AHEAD < 16:
            k_read(em, spar, i + AHEAD)
        emit_items(em, slots[2 * i])
        em(mf[1])
        emit_items(em, slots[2 * i + 1])
        if not READ_EARLY and i + AHEAD < 16:
            k_read(em, spar, i + AHEAD)
    if last:
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
    em("s_waitcnt vmcnt(0)")
    mark(em, 3)
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


def claim(em, u):
    """Wave 0, lane 0 claims a unit for the work-group: an atomic add of 1 on
    the XCD's counter whose old value lands in CLAIM while the loop runs (the
    loop's last vmcnt(0) completes it; every other lane and wave gets 0)."""
    em(f"v_mov_b32 {CLAIM}, 0")
    em(f"s_cmp_lg_u32 {S_WID}, 0")
    em(f"s_cbranch_scc1 {u}claimed")
    em(f"s_mov_b64 {S_F0}, exec")
    em("s_mov_b64 exec, 1")
    em(f"v_mov_b32 {ET[0]}, 0")
    em(f"v_mov_b32 {ET[1]}, 1")
    em("s_nop 4")
    em(f"global_atomic_add {CLAIM}, {ET[0]}, {ET[1]}, {S_CNT} sc0")
    em(f"s_mov_b64 exec, {S_F0}")
    em(f"{u}claimed:")


def block_prologue(em, paged):
    """State init, block ids of tiles 0 and 1 (inputs), QK_0.  K_0 and K_1
    are in the K buffers when the loop starts (the caller copies them in
    while the previous unit ends).  No vector memory op is issued here: the
    caller's prefetch of the next unit's query rows may still be in flight,
    and the first wait on vmcnt is the one that ends iteration 0."""
    em("s_nop 1")
    em(f"v_mov_b32 {MRUN[0]}, 0xff800000")
    em(f"v_mov_b32 {MRUN[1]}, 0xff800000")
    em(f"v_mov_b32 {LRUN[0]}, 0")
    em(f"v_mov_b32 {LRUN[1]}, 0")
    em(f"v_mov_b32 {NINF}, 0xff800000")
    em(f"v_mov_b32 {ONES}, 0x3f803f80")
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
    for i in range(AHEAD):
        k_read(em, 0, i)
    # O^T <- 0 (128 AGPRs), four writes beside each QK_0 MFMA
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
    """PV of the last tile (V and P of parity par)."""
    for i in range(AHEAD):
        v_read(em, par, i)
    for i in range(16):
        em.lds_wait(("v", i, 1))
        for x in pv_mfmas(em, i, par):
            em(x)
        if i + AHEAD < 16:
            v_read(em, par, i + AHEAD)
    em.lds_drain()


def block_kprefetch(em, u):
    """Key tiles 0 and 1 of the next unit into K buffers 0 and 1 (rows
    16 w .. 16 w + 15 of each, as the loop's fills), when S_FLAGS bit 0 is
    set.  Every wave has passed the loop's last barrier, after which no wave
    reads the K buffers."""
    em(f"s_bitcmp1_b32 {S_FLAGS}, 0")
    em(f"s_cbranch_scc0 {u}nokpf")
    for t, rs_w in ((0, S_RK_W), (1, S_RV_W)):
        lo, hi = S_NK[t]
        em(f"s_mov_b32 {rs_w[0]}, {lo}")
        em(f"s_and_b32 {rs_w[1]}, {hi}, 0xffff")
        em(f"s_mov_b32 {rs_w[2]}, {S_NREC[t]}")
        em(f"s_mov_b32 {rs_w[3]}, {RSRC_W3}")
        rsrc = S_RK if t == 0 else S_RV
        for i in range(4):
            em(f"s_add_u32 m0, {S_M0W}, {TILE * t + 1024 * i}")
            em("s_nop 0")
            em(f"buffer_load_dwordx4 {DMAK[i]}, {rsrc}, 0 offen lds")
    em(f"{u}nokpf:")


def block_output(em):
    """O^T / l as bf16 rows.  Lane (qc, h) of O[n][qb] register v holds d =
    32 n + 8 (v / 4) + 4 h + v % 4 of row qc of q-block qb: registers
    8 half .. 8 half + 7 make two 8-byte pieces, of 16-byte chunks 4 n + 2
    half (its first 4 values) and 4 n + 2 half + 1, of the lane's row half.
    v_permlane32_swap_b32 exchanges the second piece of the lanes h = 0 with
    the first piece of the lanes h = 1, so lane h holds chunk 4 n + 2 half + h
    whole, stored at row qc, byte 16 (4 n + 2 half + h).  Rows past the
    q-block's row count (the resource size) are dropped; a row without a
    visible key (l = 0) is stored as zeros."""
    em("s_nop 7")  # MFMA results (the last PV) before v_accvgpr_read
    em("s_nop 7")
    for qb in range(2):
        em(f"v_rcp_f32 {AL[qb]}, {LRUN[qb]}")
    em(f"v_cmp_lt_f32_e64 {S_F0}, 0, {LRUN[0]}")
    em(f"v_cmp_lt_f32_e64 {S_F1}, 0, {LRUN[1]}")
    em("s_nop 1")
    em(f"v_cndmask_b32_e64 {AL[0]}, 0, {AL[0]}, {S_F0}")
    em(f"v_cndmask_b32_e64 {AL[1]}, 0, {AL[1]}, {S_F1}")
    # resources of the two q-blocks' rows
    em(f"v_readfirstlane_b32 {S_RK_W[0]}, {OD[0]}")
    em(f"v_readfirstlane_b32 {S_RK_W[1]}, {OD[1]}")
    em(f"v_readfirstlane_b32 {S_RK_W[2]}, {OD[2]}")
    em(f"v_readfirstlane_b32 {S_RV_W[2]}, {OD[3]}")
    em("s_nop 4")  # VALU-written SGPRs before SALU and buffer reads
    em(f"s_add_u32 {S_RV_W[0]}, {S_RK_W[0]}, {S_ODELTA}")
    em(f"s_addc_u32 {S_RV_W[1]}, {S_RK_W[1]}, 0")
    em(f"s_and_b32 {S_RK_W[1]}, {S_RK_W[1]}, 0xffff")
    em(f"s_and_b32 {S_RV_W[1]}, {S_RV_W[1]}, 0xffff")
    em(f"s_mov_b32 {S_RK_W[3]}, {RSRC_W3}")
    em(f"s_mov_b32 {S_RV_W[3]}, {RSRC_W3}")
    t = [f"v{k}" for k in range(8)]
    groups = [8 + 4 * g for g in range(6)]  # six 4-register pieces, used in turn
    gi = 0
    for qb in range(2):
        rsrc = S_RK if qb == 0 else S_RV
        for n in range(4):
            for half in range(2):
                base = 64 + 16 * (2 * n + qb) + 8 * half
                for k in range(8):
                    em(f"v_accvgpr_read_b32 {t[k]}, a{base + k}")
                for k in range(8):
                    em(f"v_mul_f32 {t[k]}, {AL[qb]}, {t[k]}")
                g = groups[gi % len(groups)]
                gi += 1
                for e in range(4):
                    em(f"v_cvt_pk_bf16_f32 v{g + e}, {t[2 * e]}, {t[2 * e + 1]}")
                em("s_nop 1")
                em(f"v_permlane32_swap_b32 v{g}, v{g + 2}")
                em(f"v_permlane32_swap_b32 v{g + 1}, v{g + 3}")
                em("s_nop 1")
                em(f"buffer_store_dwordx4 v[{g}:{g + 3}], {OOFF}, {rsrc}, 0 offen offset:{64 * n + 32 * half}")


def program(paged):
    em = Emitter()
    u = "L%=_"
    mark(em, None)
    claim(em, u)
    block_prologue(em, paged)
    # iteration 0
    em(f"s_cmp_gt_i32 {S_JM}, 0")
    em(f"s_cbranch_scc1 {u}first")
    block_mask(em, 0)
    em(f"{u}first:")
    block_iteration(em, paged, 0, True, f"{u}i0")
    em.lds = []
    em(f"s_mov_b32 {S_J}, 1")
    em(f"{u}top:")
    for par in (1, 0):
        em(f"s_cmp_gt_i32 {S_J}, {S_LAST}")
        em(f"s_cbranch_scc1 {u}final")
        em(f"s_cmp_lt_i32 {S_J}, {S_JM}")
        em(f"s_cbranch_scc1 {u}nomask{par}")
        block_mask(em, par)
        em(f"{u}nomask{par}:")
        em(f"s_cmp_eq_u32 {S_J}, {S_LAST}")
        em(f"s_cbranch_scc1 {u}last{par}")
        block_iteration(em, paged, par, False, f"{u}f{par}")
        em.lds = []
        em(f"s_add_u32 {S_J}, {S_J}, 1")
    em(f"s_branch {u}top")
    # the unit's last iteration (j = S_LAST >= 1), out of line
    for par in (1, 0):
        em(f"{u}last{par}:")
        block_iteration(em, paged, par, False, f"{u}l{par}", last=True)
        em.lds = []
        em(f"s_branch {u}final")
    # out-of-line slow paths
    block_slow(em, 0, f"{u}i0")
    for par in (1, 0):
        block_slow(em, par, f"{u}f{par}")
        block_slow(em, par, f"{u}l{par}")
    em(f"{u}final:")
    em("s_waitcnt vmcnt(0) lgkmcnt(0)")
    em.lds = []
    block_kprefetch(em, u)
    em(f"s_bitcmp1_b32 {S_LAST}, 0")
    em(f"s_cbranch_scc1 {u}final1")
    block_pv_only(em, 0)
    em(f"s_branch {u}done")
    em(f"{u}final1:")
    block_pv_only(em, 1)
    em(f"{u}done:")
    # l_run of the lane's row over both key halves (lanes l and l ^ 32)
    for qb in range(2):
        em(f"v_mov_b32 {ET[qb]}, {LRUN[qb]}")
    em("s_nop 1")
    for qb in range(2):
        em(f"v_permlane32_swap_b32 {LRUN[qb]}, {ET[qb]}")
    for qb in range(2):
        em(f"v_add_f32 {LRUN[qb]}, {LRUN[qb]}, {ET[qb]}")
    mark(em, 6)
    block_output(em)
    em("s_nop 7")
    em("s_nop 7")
    em("s_nop 3")
    return em.lines


CLOBBERS = (
    [f"v{i}" for i in range(0, 192)] + [f"v{i}" for i in range(216, 220)] + [f"v{i}" for i in range(222, 243)]
    + [f"a{i}" for i in range(64, 256)] + [f"s{i}" for i in range(64, 100)]
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
    clob = ", ".join(f'"{c}"' for c in CLOBBERS)
    text = [
        "// Generated by gen_prefill_mx.py; do not edit by hand.",
        "// The tile loop of one prefill work item (see paged_prefill_mx.hip).",
        "#pragma once",
        "",
        render("NVS_PREFILL_MX_ASM_PAGED", paged),
        "",
        render("NVS_PREFILL_MX_ASM_LOCAL", local),
        "",
        f"#define NVS_PREFILL_MX_CLOBBERS {clob}",
        "",
    ]
    path = os.path.join(here, "prefill_mx_asm.inc")
    with open(path, "w") as f:
        f.write("\n".join(text))
    print(f"wrote {path}: {len(paged)} + {len(local)} lines", file=sys.stderr)


if __name__ == "__main__":
    main()
