#!/usr/bin/env python3
"""Whole-program CPU check of the generated prefill tile loop
(prefill_mx_asm.inc) for its LDS synchronisation and its tile order.

The program is run, one wave at a time, by an interpreter of its scalar and
lane instructions over random batches (block tables with missing and
out-of-pool blocks, rows without keys, one-tile units, fewer keys than rows,
the slow path taken at random), claiming units from a modelled counter as
the kernel does.  Every wave of a work-group runs the same control flow, so
one trace stands for all four, with:
  * race rules for the shared K and V tile buffers (every wave reads whole
    tiles, each fills 16 rows of each): a read needs the region's last fill
    completed by a vmcnt wait and a barrier after that wait; a fill needs
    every read of the region's old content completed by an lgkmcnt wait and
    a barrier after that; the wave's own query stage needs the waits alone;
  * a check of what the MFMAs read: the K operands of each QK^T tile (32
    MFMAs) and the V operands of each PV tile come from one fill of one
    buffer, and the tiles read, in order, are each claimed unit's tiles in
    order (the plan records are modelled on schedule.hip's plan kernel).
Every buffer load and store is checked to use a raw resource (word 3) with
no stride and a 48-bit base.  The arithmetic of scores and outputs is not
interpreted.  Run by the build
with a few batches; `python check_prefill_lds.py SEED BATCHES` runs more."""
import importlib.util
import os
import random
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
spec = importlib.util.spec_from_file_location("gen_prefill_mx", os.path.join(HERE, "gen_prefill_mx.py"))
G = importlib.util.module_from_spec(spec)
spec.loader.exec_module(G)

M32 = 0xFFFFFFFF
_HIP = open(os.path.join(HERE, "paged_prefill_mx.hip")).read()
QSTAGE = int(re.search(r"constexpr int kMxQStage = (\d+);", _HIP).group(1))  # the query stage's LDS offset
NB = 5000            # blocks in the modelled pool
SLOT_LDS = 1 << 20   # the claim slots' LDS address (past every tile region)


def s32(x):
    x &= M32
    return x - (1 << 32) if x & 0x80000000 else x


class Fail(Exception):
    pass


class Sim:
    """One wave's run of the program: scalar and lane state, the outstanding
    vector-memory and LDS operations, barriers, and each LDS region's fills
    and reads."""

    def __init__(self, lines, w, rng, slow_p):
        self.lines = lines
        self.labels = {ln[:-1]: i for i, ln in enumerate(lines) if ln.endswith(":")}
        self.s, self.v = {}, {}
        self.scc = 0
        self.m0 = 0
        self.exec1 = False
        self.w = w
        self.rng = rng
        self.slow_p = slow_p
        self.pos = 0
        self.vmq, self.lgq = [], []  # outstanding ops (dicts), issue order
        self.barriers = []
        self.regions = {}  # region -> {"reads": [reads of its content], "content": id, "fills": [in flight]}
        self.slots = {}  # ring slot register base -> (region, content)
        self.claim_lds = {}
        self.counter = 3
        self.qk, self.pv = [], []  # operand contents of QK / PV MFMAs

    # ---------------------------------------------------------- registers
    def sget(self, tok):
        tok = tok.strip()
        if tok.startswith("0x") or tok.startswith("-0x"):
            return int(tok, 16) & M32
        if re.fullmatch(r"-?\d+", tok):
            return int(tok) & M32
        if re.fullmatch(r"-?\d+\.\d+", tok):
            return 0
        if tok == "m0":
            return self.m0
        m = re.fullmatch(r"s(\d+)", tok)
        if m:
            return self.s.get(int(m.group(1)), 0xDEADBEEF)
        if tok == "vcc":
            return self.s.get("vcc", 0)
        raise ValueError(tok)

    def sset(self, tok, val):
        tok = tok.strip()
        if tok == "m0":
            self.m0 = val & M32
            return
        m = re.fullmatch(r"s(\d+)", tok)
        self.s[int(m.group(1))] = val & M32

    def pair(self, tok):
        tok = tok.strip()
        if tok == "exec":
            return 1 if self.exec1 else M32 | (M32 << 32)
        if tok == "vcc":
            return self.s.get("vcc", 0)
        if re.fullmatch(r"-?\d+", tok):
            return int(tok) & ((1 << 64) - 1)
        m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
        a = int(m.group(1))
        return self.s.get(a, 0) | (self.s.get(a + 1, 0) << 32)

    def pset(self, tok, val):
        tok = tok.strip()
        if tok == "exec":
            self.exec1 = (val == 1)
            return
        if tok == "vcc":
            self.s["vcc"] = val
            return
        m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
        a = int(m.group(1))
        self.s[a] = val & M32
        self.s[a + 1] = (val >> 32) & M32

    def vget(self, tok):
        return self.v.setdefault(tok.strip(), [0] * 64)

    def vsrc(self, tok):
        tok = tok.strip()
        if re.fullmatch(r"v\d+", tok):
            return self.vget(tok)
        return [self.sget(tok)] * 64

    # ------------------------------------------------------- LDS regions
    def region_of(self, addr):
        if addr >= SLOT_LDS:
            return ("slot",)
        if addr >= QSTAGE:
            w = (addr - QSTAGE) // 16384
            assert w == self.w, (addr, self.w)
            return ("q", (addr - QSTAGE - 16384 * w) // 8192)  # the stage's two q-block halves
        return ("t", addr // 16384)

    def fill_region(self, m0):
        a = m0 - 4096 * self.w
        if m0 >= QSTAGE:
            return self.region_of(m0)
        assert 0 <= a < QSTAGE, m0
        return ("t", a // 16384)

    def fail(self, msg):
        raise Fail(f"pos {self.pos} line {self.pc - 1} [{self.lines[self.pc - 1]}]: {msg}")

    def barrier_between(self, a, b):
        return any(a < x < b for x in self.barriers)

    def lds_read(self, dst, addr):
        reg = self.region_of(addr)
        op = {"pos": self.pos, "done": None, "region": reg}
        self.lgq.append(op)
        if reg[0] == "slot":
            return op
        st = self.regions.setdefault(reg, {"reads": [], "content": None, "fills": []})
        for f in st["fills"]:
            if f["done"] is None:
                self.fail(f"read of {reg} while a fill of it (pos {f['pos']}) is not waited")
            if reg[0] == "t" and not self.barrier_between(f["done"], self.pos):
                self.fail(f"read of {reg}: no barrier after its fill's wait (fill pos {f['pos']}, wait {f['done']})")
        st["reads"].append(op)
        if dst is not None:
            self.slots[dst] = (reg, st["content"])
        return op

    def lds_fill(self, m0, content):
        reg = self.fill_region(m0)
        op = {"pos": self.pos, "done": None, "region": reg}
        self.vmq.append(op)
        st = self.regions.setdefault(reg, {"reads": [], "content": None, "fills": []})
        for r in st["reads"]:
            if r["done"] is None:
                self.fail(f"fill of {reg} while a read of it (pos {r['pos']}) is not waited")
            if reg[0] == "t" and not self.barrier_between(r["done"], self.pos):
                self.fail(f"fill of {reg}: no barrier after the wait of a read of its old content (read {r['pos']})")
        st["reads"] = []
        # fills of one region with a content other than the one in flight must follow its completion
        for f in st["fills"]:
            if f["done"] is None and f["content"] != content:
                self.fail(f"fill of {reg} with {content} while a fill with {f['content']} is in flight")
        op["content"] = content
        st["fills"] = [f for f in st["fills"] if f["done"] is None] + [op]
        st["content"] = content
        return op

    def lds_write(self, addr):
        reg = self.region_of(addr)
        self.lgq.append({"pos": self.pos, "done": None, "region": reg})
        st = self.regions.get(reg)
        if st and reg[0] != "slot":
            for f in st["fills"]:
                if f["done"] is None:
                    self.fail(f"write of {reg} while a fill of it is not waited")

    def waitcnt(self, args):
        txt = " ".join(args)
        m = re.search(r"vmcnt\((\d+)\)", txt)
        if m:
            n = int(m.group(1))
            for op in self.vmq[:max(0, len(self.vmq) - n)]:
                if op["done"] is None:
                    op["done"] = self.pos
            self.vmq = self.vmq[max(0, len(self.vmq) - n):]
        m = re.search(r"lgkmcnt\((\d+)\)", txt)
        if m:
            n = int(m.group(1))
            for op in self.lgq[:max(0, len(self.lgq) - n)]:
                if op["done"] is None:
                    op["done"] = self.pos
            self.lgq = self.lgq[max(0, len(self.lgq) - n):]

    # --------------------------------------------------------------- run
    def run(self, max_steps=5_000_000):
        pc = 0
        for _ in range(max_steps):
            if pc >= len(self.lines):
                return
            ln = self.lines[pc]
            pc += 1
            self.pc = pc
            self.pos += 1
            if ln.endswith(":"):
                continue
            op, _, rest = ln.partition(" ")
            args = [x.strip() for x in re.split(r",(?![^\[]*\])", rest)] if rest else []
            if op == "s_nop":
                continue
            if op == "s_barrier":
                self.barriers.append(self.pos)
                continue
            if op == "s_waitcnt":
                self.waitcnt(args)
                continue
            if op == "s_branch":
                pc = self.labels[args[0]]
                continue
            if op in ("s_cbranch_scc1", "s_cbranch_scc0"):
                if (self.scc == 1) == (op == "s_cbranch_scc1"):
                    pc = self.labels[args[0]]
                continue
            self.exec_op(op, args, ln)
        raise RuntimeError("too many steps")

    def exec_op(self, op, args, ln):
        if op == "s_mov_b32":
            self.sset(args[0], self.sget(args[1]))
        elif op in ("s_add_u32", "s_add_i32"):
            r = self.sget(args[1]) + self.sget(args[2])
            self.scc = int(r > M32) if op == "s_add_u32" else 0
            self.sset(args[0], r)
        elif op == "s_addc_u32":
            r = self.sget(args[1]) + self.sget(args[2]) + self.scc
            self.scc = int(r > M32)
            self.sset(args[0], r)
        elif op in ("s_sub_u32", "s_sub_i32"):
            a, b = self.sget(args[1]), self.sget(args[2])
            self.scc = int(b > a) if op == "s_sub_u32" else 0
            self.sset(args[0], a - b)
        elif op == "s_mul_i32":
            self.sset(args[0], s32(self.sget(args[1])) * s32(self.sget(args[2])))
        elif op == "s_mul_hi_u32":
            self.sset(args[0], (self.sget(args[1]) * self.sget(args[2])) >> 32)
        elif op == "s_lshl_b32":
            r = self.sget(args[1]) << (self.sget(args[2]) & 31)
            self.sset(args[0], r)
            self.scc = int(r & M32 != 0)
        elif op == "s_lshr_b32":
            r = self.sget(args[1]) >> (self.sget(args[2]) & 31)
            self.sset(args[0], r)
            self.scc = int(r != 0)
        elif op == "s_ashr_i32":
            r = s32(self.sget(args[1])) >> (self.sget(args[2]) & 31)
            self.sset(args[0], r)
            self.scc = int(r != 0)
        elif op == "s_and_b32":
            r = self.sget(args[1]) & self.sget(args[2])
            self.sset(args[0], r)
            self.scc = int(r != 0)
        elif op in ("s_min_i32", "s_max_i32"):
            f = min if op == "s_min_i32" else max
            self.sset(args[0], f(s32(self.sget(args[1])), s32(self.sget(args[2]))))
        elif op in ("s_min_u32", "s_max_u32"):
            f = min if op == "s_min_u32" else max
            self.sset(args[0], f(self.sget(args[1]), self.sget(args[2])))
        elif op.startswith("s_cmp_"):
            kind, ty = op[6:].rsplit("_", 1)
            a, b = self.sget(args[0]), self.sget(args[1])
            if ty == "i32":
                a, b = s32(a), s32(b)
            self.scc = int({"eq": a == b, "lg": a != b, "lt": a < b, "le": a <= b, "gt": a > b,
                            "ge": a >= b}[kind])
        elif op == "s_cselect_b32":
            self.sset(args[0], self.sget(args[1]) if self.scc else self.sget(args[2]))
        elif op == "s_cselect_b64":
            self.pset(args[0], self.pair(args[1]) if self.scc else self.pair(args[2]))
        elif op == "s_bitcmp1_b32":
            self.scc = (self.sget(args[0]) >> self.sget(args[1])) & 1
        elif op == "s_mov_b64":
            self.pset(args[0], self.pair(args[1]))
        elif op == "s_or_b64":
            r = self.pair(args[1]) | self.pair(args[2])
            self.pset(args[0], r)
            self.scc = int(r != 0)
        elif op == "v_readlane_b32":
            self.sset(args[0], self.vget(args[1])[int(args[2])])
        elif op == "v_readfirstlane_b32":
            self.sset(args[0], self.vget(args[1])[0])
        elif op == "v_writelane_b32":
            self.vget(args[0])[int(args[2])] = self.sget(args[1])
        elif op == "v_mov_b32":
            if self.exec1:
                self.vget(args[0])[0] = self.vsrc(args[1])[0]
            else:
                self.v[args[0]] = list(self.vsrc(args[1]))
        elif op == "v_add_u32":
            self.v[args[0]] = [(x + y) & M32 for x, y in zip(self.vsrc(args[1]), self.vsrc(args[2]))]
        elif op == "v_subrev_u32":
            self.v[args[0]] = [(y - x) & M32 for x, y in zip(self.vsrc(args[1]), self.vsrc(args[2]))]
        elif op == "v_xor_b32":
            self.v[args[0]] = [(x ^ y) & M32 for x, y in zip(self.vsrc(args[1]), self.vsrc(args[2]))]
        elif op == "v_mbcnt_lo_u32_b32":
            self.v[args[0]] = [min(l, 32) for l in range(64)]
        elif op == "v_mbcnt_hi_u32_b32":
            self.v[args[0]] = list(range(64))
        elif op == "v_lshlrev_b32":
            sh = self.sget(args[1])
            self.v[args[0]] = [(x << sh) & M32 for x in self.vsrc(args[2])]
        elif op == "v_cmp_nge_f32":  # the tile's row sums: sometimes take the slow path
            self.s["vcc"] = 1 if self.rng.random() < self.slow_p else 0
        elif op.startswith("v_cmp_neq_f32"):  # alpha != 1 somewhere
            self.pset(args[0], 1 if self.rng.random() < 0.5 else 0)
        elif op.startswith("v_cmp_eq_f32"):  # running max still -inf: never
            self.pset(args[0], 0)
        elif op.startswith("v_cmp"):
            dst = args[0]
            if dst.startswith("s[") or dst == "vcc":
                self.pset(dst, 0)
        elif op.startswith("v_mfma"):
            a = args[1]
            m = re.fullmatch(r"a\[(\d+):(\d+)\]", a)
            if m:
                base = int(m.group(1))
                if 224 <= base < 256:
                    self.qk.append(self.slots.get(base))
                elif 192 <= base < 224:
                    self.pv.append(self.slots.get(base))
        elif op.startswith("v_"):
            pass  # arithmetic of the scores and outputs: no control flow
        elif op == "ds_read_b128":
            addr = self.vget(args[1].split()[0])[0] + self.off(args)
            dst = args[0]
            m = re.fullmatch(r"a\[(\d+):(\d+)\]", dst)
            self.lds_read(int(m.group(1)) if m and int(m.group(1)) >= 192 else None, addr)
        elif op == "ds_read_b64_tr_b16":
            addr = self.vget(args[1].split()[0])[0] + self.off(args)
            m = re.fullmatch(r"a\[(\d+):(\d+)\]", args[0])
            base = int(m.group(1))
            slot = 192 + 4 * ((base - 192) // 4)
            o = self.lds_read(None, addr)
            reg = o["region"]
            content = (reg, self.regions[reg]["content"])
            if base % 4 == 0:
                self.half = content
            else:
                if self.half != content:
                    self.fail("the two halves of a V operand read different tiles")
                self.slots[slot] = content
        elif op == "ds_read_b32":
            addr = self.vget(args[1].split()[0])[0] + self.off(args)
            self.lds_read(None, addr)
            self.vget(args[0])[0] = self.claim_lds.get(addr, 0)
            self.v[args[0]] = [self.claim_lds.get(addr, 0)] * 64
        elif op == "ds_write_b32":
            addr = self.vget(args[0])[0] + self.off(args)
            self.lds_write(addr)
            self.claim_lds[addr] = self.vget(args[1])[0]
        elif op == "ds_write_b128":
            addr = self.vget(args[0])[0] + self.off(args)
            self.lds_write(addr)
        elif op == "buffer_load_dword":
            rs = args[2]
            r0 = self.check_rsrc(rs)
            base = self.s[r0] | ((self.s[r0 + 1] & 0xFFFF) << 32)
            nrec = self.s[r0 + 2]
            voff = self.vget(args[1])
            self.vmq.append({"pos": self.pos, "done": None, "region": None})
            if rs == G.S_RREC:
                idx = (base - self.rec_base) // 64
                assert (base - self.rec_base) % 64 == 0 and 0 <= idx < len(self.records), (base, idx)
                self.v[args[0]] = [self.records[idx][k] & M32 if voff[k] < nrec and k < 16 else 0 for k in range(64)]
            elif rs == G.S_RBT:
                o = voff[0]
                val = self.mem32.get(base + o, 0) if o + 4 <= nrec else 0
                self.v[args[0]] = [val & M32] * 64
            else:
                raise NotImplementedError(ln)
        elif op == "buffer_load_dwordx4":
            r0 = self.check_rsrc(args[1])
            base = self.s[r0] | ((self.s[r0 + 1] & 0xFFFF) << 32)
            nrec = self.s[r0 + 2]
            assert args[-1].endswith("lds"), ln
            self.lds_fill(self.m0, (base, nrec) if nrec else ("zero",))
        elif op == "buffer_store_dwordx4":
            self.check_rsrc(args[2])
            self.vmq.append({"pos": self.pos, "done": None, "region": None})
        elif op == "global_atomic_add":
            self.vmq.append({"pos": self.pos, "done": None, "region": None})
            assert self.exec1
            self.vget(args[0])[0] = self.counter
            self.counter += 1
        else:
            raise NotImplementedError(op)

    def check_rsrc(self, tok):
        """A buffer resource as the loop must build it: raw (word 3), no
        stride and a 48-bit base (word 1's high half zero)."""
        m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
        r0 = int(m.group(1))
        w1, w3 = self.s.get(r0 + 1, 0xDEADBEEF), self.s.get(r0 + 3, 0xDEADBEEF)
        if w3 != int(G.RSRC_W3, 16) or w1 >> 16:
            self.fail(f"buffer resource {tok}: word 1 {w1:#x}, word 3 {w3:#x}")
        return r0

    @staticmethod
    def off(args):
        m = re.search(r"offset:(\d+)", " ".join(args))
        return int(m.group(1)) if m else 0


# ------------------------------------------------------------------ model
def plan_records(seqs, pbm, ntq, paged, bs, bt_stride, Tk, cu_k0, bt_rows):
    recs = []
    q0 = 0
    for b, (L, K, blks) in enumerate(seqs):
        np_ = min((L + pbm - 1) // pbm, ntq)
        k0 = cu_k0[b]
        for i in range(np_):
            qt = np_ - 1 - i
            p0 = qt * pbm
            p_last = min(L, p0 + pbm) - 1
            off = K - L
            kv_end = min(K, p_last + off + 1)
            nt = (kv_end + 63) // 64 if (p0 < L and kv_end > 0) else 0

            def tb(t):
                lb = 64 * t // bs
                nblk = min((K + bs - 1) // bs, bt_stride)
                x = blks[lb] if lb < nblk else -1
                return x if 0 <= x < NB else -1  # the plan's check against the pool
            if paged:
                k0c, kf = 0, K
                btb = 4 * min((K + bs - 1) // bs, bt_stride)
                bb = (tb(0), tb(1), tb(2))
            else:
                k0c = min(max(k0, 0), Tk)
                kf = max(0, min(K, Tk - k0c))
                btb = 0
                bb = (-1, -1, -1)
            recs.append([b * ntq + qt, q0, L, k0, K, *bb, p0, nt, kf, off, k0c, b, btb, 0])
        q0 += L
    return recs


def unit_tiles(u, recs, a, seqs, NB):
    """(K tiles, V tiles) of unit u as (address, bytes) with bytes > 0 only."""
    pe = a["Hkv"] * a["hgroups"]
    idx, rem = divmod(u, pe)
    hkv, hg = divmod(rem, a["hgroups"])
    item, q0, L, k0, K = recs[idx][:5]
    b, qt = divmod(item, a["ntq"])
    p0 = qt * a["pbm"]
    nt = 0
    if p0 < L:
        p_last = min(L, p0 + a["pbm"]) - 1
        kv_end = min(K, p_last + (K - L) + 1)
        nt = (kv_end + 63) // 64 if kv_end > 0 else 0
    out = ([], [])
    M48 = (1 << 48) - 1
    # a unit of one tile runs the QK^T of tile 1 too (its scores unused)
    for t in range(nt + (1 if nt == 1 else 0)):
        phantom = t >= nt
        if a["paged"]:
            krow = a["Hkv"] * 256
            lb = 64 * t // a["bs"]
            nblk = min((K + a["bs"] - 1) // a["bs"], a["bt_stride"])
            blk = seqs[b][2][lb] if lb < nblk else -1
            if blk < 0 or blk >= NB:
                continue
            rows = min(max(K - 64 * t, 0), 64)
            first = (blk * a["bs"] + (64 * t) % a["bs"]) * krow
            if rows == 0:
                continue
            for k, base in enumerate((a["kc"], a["vc"])):
                if not (phantom and k == 1):
                    out[k].append(((base + hkv * 256 + first) & M48, rows * krow))
        else:
            k0c = min(max(k0, 0), a["Tk"])
            krows = max(0, min(K, a["Tk"] - k0c))
            rows = min(max(krows - 64 * t, 0), 64)
            if rows == 0:
                continue
            for k, (base, ts, hs) in enumerate(((a["k"], a["k_ts"], a["k_hs"]), (a["v"], a["v_ts"], a["v_hs"]))):
                addr = base + (k0c * ts + hkv * hs) * 2 + 64 * t * ts * 2
                if not (phantom and k == 1):
                    out[k].append((addr & M48, rows * ts * 2))
    return out


def groups(ops, what):
    tiles = []
    for k in range(0, len(ops), 32):
        g = ops[k:k + 32]
        if len(g) < 32:
            raise Fail(f"{what}: a tile of {len(g)} MFMAs")
        if any(x != g[0] for x in g):
            raise Fail(f"{what}: one tile's MFMAs read different buffers/fills: {set(map(str, g))}")
        tiles.append(g[0])
    return tiles


def check_case(rng, paged, slow_p):
    Hkv = rng.choice([1, 2, 3, 5, 8])
    g = rng.choice([1, 2, 3, 4, 5, 8, 16])
    Hq = Hkv * g
    hpi = 1
    while 2 * hpi <= g and 2 * hpi <= 8:
        hpi *= 2
    hgroups = (g + hpi - 1) // hpi
    pbm = 256 // hpi
    bs = rng.choice([64, 128, 256]) if paged else 64
    B = rng.randint(1, 5)
    seqs = []
    for _ in range(B):
        L = rng.randint(1, 600)
        P = rng.choice([0, 0, bs * rng.randint(0, 3), rng.randint(0, 300)]) if paged else rng.choice([0, 0, 3])
        K = L + P if rng.random() < 0.85 else max(0, L - rng.randint(1, L))
        nb = (K + bs - 1) // bs
        blks = [rng.randrange(NB) if rng.random() > 0.04 else rng.choice([-1, NB + 7]) for _ in range(nb + 2)]
        seqs.append((L, K, blks))
    ntq = max((L + pbm - 1) // pbm for L, _, _ in seqs)
    bt_stride = max(len(bl) for _, _, bl in seqs) + rng.randint(0, 3)
    Tk = sum(K for _, K, _ in seqs) - (rng.randint(0, 40) if not paged else 0)
    cu_k0, acc = [], 0
    for _, K, _ in seqs:
        cu_k0.append(acc)
        acc += K
    base = lambda: rng.randrange(1 << 40, 1 << 46) & ~255
    a = dict(Hkv=Hkv, hgroups=hgroups, hpi=hpi, g=g, Hq=Hq, ntq=ntq, pbm=pbm, paged=paged, bs=bs,
             bt_stride=bt_stride, Tk=Tk, kc=base(), vc=base(), k=base(), v=base(), k_ts=Hkv * 128,
             v_ts=Hkv * 128, k_hs=128, v_hs=128, q=base(), q_ts=Hq * 128, q_hs=128, out=base(),
             out_ts=Hq * 128, out_hs=128, bt=base())
    recs = plan_records(seqs, pbm, ntq, paged, bs, bt_stride, Tk, cu_k0, None)
    pe = Hkv * hgroups
    units = len(recs) * pe
    lines = G.program(paged)
    w = rng.randrange(4)
    xcd = rng.randrange(8)
    sim = Sim(lines, w, rng, slow_p)
    sim.records = recs
    sim.rec_base = base()
    sim.mem32 = {}
    if paged:
        for b, (_, _, blks) in enumerate(seqs):
            for k, x in enumerate(blks[:bt_stride]):
                sim.mem32[a["bt"] + b * bt_stride * 4 + 4 * k] = x & M32
    krow = Hkv * 256 if paged else a["k_ts"] * 2
    qrts = a["q_ts"] * 2
    mpe = 0 if pe == 1 else ((1 << 32) + pe - 1) // pe
    claims = [0, 1, 2]
    u0, u1, u2 = (8 * c + xcd for c in claims)
    if u0 >= units:
        return 0
    for name, val in (("S_KROW", krow), ("S_BS", bs), ("S_NB", NB), ("S_M0W", 4096 * w),
                      ("S_SCALE", 0), ("S_WID", 0), ("S_QST", QSTAGE + 16384 * w),
                      ("S_QD", QSTAGE + 16384 * w), ("S_XCD", xcd), ("S_NUNITS", units), ("S_MPE", mpe),
                      ("S_PE", pe), ("S_REC_LO", sim.rec_base & M32), ("S_REC_HI", sim.rec_base >> 32),
                      ("S_Q16", 16 * qrts), ("S_SLOT", SLOT_LDS), ("S_U0", u0), ("S_U1", u1),
                      ("S_PE1", M32 if pe == 1 else 0), ("S_U2IN", u2), ("S_O4", 4 * a["out_ts"] * 2)):
        sim.sset(getattr(G, name), val)
    sim.s[10], sim.s[11] = 0x1000, 0  # the counter address (the model's counter)
    bank = [0] * 64
    vals = {0: hgroups - 1, 1: hpi, 2: g, 3: Hq - 1}
    for qb in range(2):
        qbi = 2 * w + qb
        vals[4 + qb] = qbi % hpi
        vals[6 + qb] = 32 * (qbi // hpi)

    def put64(k, p):
        vals[k] = p & M32
        vals[k + 1] = p >> 32
    put64(8, a["kc"] if paged else a["k"])
    put64(10, a["vc"] if paged else a["v"])
    vals[12] = 0 if paged else a["k_ts"] * 2
    vals[13] = 256 if paged else a["k_hs"] * 2
    vals[14] = 256 if paged else a["v_hs"] * 2
    put64(15, a["q"])
    vals[17] = qrts
    vals[18] = a["q_hs"] * 2
    put64(19, a["out"])
    vals[21] = a["out_ts"] * 2
    vals[22] = a["out_hs"] * 2
    put64(23, a["bt"] if paged else 0)
    vals[25] = 4 * bt_stride if paged else 0
    for k, x in vals.items():
        bank[k] = x & M32
    sim.v[G.BANKC] = bank
    sim.v[G.LANEC] = [((l & 31) - 4 * (l >> 5)) & M32 for l in range(64)]
    for st in range(8):
        sim.v[G.KADDR[st]] = [32 * st] * 64
    vb0 = G.LDS_V0 + (G.NVBUF - 1) * G.TILE  # the C++ side starts them in the last V buffer
    for n in range(4):
        for e in range(2):
            sim.v[G.VADDR[(n, e)]] = [vb0 + 8 * e * 256 + 64 * n] * 64
    sim.v[G.RL] = [QSTAGE + 16384 * w] * 64
    sim.run()
    # the units in claim order that have tiles
    order = [u0, u1, u2] + [8 * c + xcd for c in range(3, sim.counter)]
    order = [u for u in order if u < units]
    expk, expv = [], []
    for u in order:
        kt, vt = unit_tiles(u, recs, a, seqs, NB)
        expk += kt
        expv += vt
    gotk = [c[1] for c in groups(sim.qk, "QK") if c[1] != ("zero",)]
    gotv = [c[1] for c in groups(sim.pv, "PV") if c[1] != ("zero",)]
    if gotk != expk:
        raise Fail(f"K tile sequence differs: got {len(gotk)} want {len(expk)}; first diff at "
                   f"{next((i for i, (x, y) in enumerate(zip(gotk, expk)) if x != y), min(len(gotk), len(expk)))}")
    if gotv != expv:
        raise Fail(f"V tile sequence differs: got {len(gotv)} want {len(expv)}; first diff at "
                   f"{next((i for i, (x, y) in enumerate(zip(gotv, expv)) if x != y), min(len(gotv), len(expv)))}")
    return len(order)


def main(seed=0, batches=40):
    rng = random.Random(seed)
    n = units = 0
    for _ in range(batches):
        for paged in (True, False):
            units += check_case(rng, paged, slow_p=rng.choice([0.0, 0.05, 0.3]))
            n += 1
    return n, units


if __name__ == "__main__":
    seed = int(sys.argv[1]) if len(sys.argv) > 1 else 0
    batches = int(sys.argv[2]) if len(sys.argv) > 2 else 2
    try:
        n, units = main(seed, batches)
    except Fail as e:
        print(f"prefill loop LDS check failed: {e}", file=sys.stderr)
        sys.exit(1)
    print(f"{n} batches, {units} units: no LDS race; every QK^T / PV tile read its unit's tile from one fill")
