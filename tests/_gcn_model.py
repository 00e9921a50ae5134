"""Test infrastructure: a functional model of the gfx950 instructions the generated prefill
kernel body (gguf_train_amd/csrc/prefill_asm_gen.py) uses, so that its control flow, waits and
results can be checked on the CPU.

Per-wave state (VGPR/AGPR/SGPR, exec, vcc, scc, m0), LDS of the workgroup, a flat global memory
made of named numpy buffers at fake addresses.  Asynchronous operations are modelled so that
missing waits show up as errors:
  - LDS reads (ds_read*) land at the s_waitcnt lgkmcnt that retires them; reading a destination
    register before that raises;
  - global loads and LDS DMA (global_load_lds) land at s_waitcnt vmcnt; LDS bytes with a DMA in
    flight raise when read; registers with a load in flight raise when read.
Waves run round robin between barriers; a barrier that not every live wave reaches, or a wave
ending while others wait, raises (deadlock).  MFMA hazards and timing are not modelled.
"""
import re
import struct

import numpy as np

F16 = np.float16


class EmuError(Exception):
    pass


def f32(u):
    return np.asarray(u, np.uint32).view(np.float32)


def u32(f):
    return np.asarray(f, np.float32).view(np.uint32)


class Memory:
    def __init__(self):
        self.bufs = []  # (base, bytearray-like numpy uint8)
        self.next = 0x100000

    def alloc(self, name, arr):
        data = np.frombuffer(np.ascontiguousarray(arr).tobytes(), np.uint8).copy()
        base = self.next
        self.bufs.append([base, data, name])
        self.next += (len(data) + 0xFFFF) & ~0xFFF
        self.next += 0x10000
        return base

    def find(self, addr, n):
        for b in self.bufs:
            if b[0] <= addr and addr + n <= b[0] + len(b[1]):
                return b
        raise EmuError(f"global access out of bounds: addr {addr:#x} size {n}")

    def read(self, addr, n):
        b = self.find(addr, n)
        o = addr - b[0]
        return b[1][o:o + n]

    def write(self, addr, data):
        b = self.find(addr, len(data))
        o = addr - b[0]
        b[1][o:o + len(data)] = data

    def get(self, name):
        for b in self.bufs:
            if b[2] == name:
                return b[1]


def parse(lines):
    """-> (instrs [(op, args, text)], labels {name: index})"""
    instrs, labels = [], {}
    for l in lines:
        l = l.strip()
        if not l:
            continue
        if l.endswith(":") and " " not in l:
            labels[l[:-1]] = len(instrs)
            continue
        parts = l.split(None, 1)
        op = parts[0]
        args = [a.strip() for a in re.split(r",(?![^\[]*\])", parts[1])] if len(parts) > 1 else []
        instrs.append((op, args, l))
    return instrs, labels


def reg_range(tok):
    """'v12' -> ('v', 12, 1); 'v[4:7]' -> ('v', 4, 4); 'a[0:15]' -> ('a', 0, 16)"""
    m = re.fullmatch(r"([vas])\[(\d+):(\d+)\]", tok)
    if m:
        return m.group(1), int(m.group(2)), int(m.group(3)) - int(m.group(2)) + 1
    m = re.fullmatch(r"([vas])(\d+)", tok)
    if m:
        return m.group(1), int(m.group(2)), 1
    return None


class Wave:
    def __init__(self, wid, nwaves):
        self.wid = wid
        self.v = np.zeros((256, 64), np.uint32)
        self.a = np.zeros((256, 64), np.uint32)
        self.s = np.zeros(128, np.uint32)
        self.exec = np.ones(64, bool)
        self.vcc = np.zeros(64, bool)
        self.scc = 0
        self.m0 = 0
        self.pc = 0
        self.done = False
        self.at_barrier = False
        self.lgkm = []   # pending LDS reads: (dst kind, base, n regs, values[n,64])
        self.vm = []     # pending global loads / DMA: ('reg', kind, base, vals) or ('lds', addrs, bytes)
        self.pending_regs = {}  # (kind, idx) -> count
        self.count = 0


class Emu:
    def __init__(self, instrs, labels, mem, nwaves, lds_bytes, operands, max_steps=5_000_000):
        self.ins, self.labels, self.mem = instrs, labels, mem
        self.lds = np.zeros(lds_bytes, np.uint8)
        self.lds_pending = np.zeros(lds_bytes, np.int32)
        self.waves = [Wave(w, nwaves) for w in range(nwaves)]
        self.ops = operands  # {'%[name]': ('s', value) or ('s64', value)}
        self.max_steps = max_steps
        self.trace_counts = {}

    # ---- operand access
    def sub(self, tok):
        for k, v in self.ops.items():
            if tok == k:
                return v
        return None

    def rd_s(self, w, tok):
        """scalar source -> python int (32-bit) or 64-bit for s[x:y]"""
        o = self.sub(tok)
        if o is not None:
            return o
        r = reg_range(tok)
        if r:
            k, i, n = r
            assert k == "s", tok
            if n == 1:
                return int(w.s[i])
            return int(w.s[i]) | (int(w.s[i + 1]) << 32)
        if tok == "m0":
            return w.m0
        if tok == "vcc":
            return self.mask_int(w.vcc)
        if tok == "exec":
            return self.mask_int(w.exec)
        return self.const(tok) & 0xFFFFFFFF

    def const(self, tok):
        fl = {"0.5": 0x3F000000, "-0.5": 0xBF000000, "1.0": 0x3F800000, "-1.0": 0xBF800000,
              "2.0": 0x40000000, "-2.0": 0xC0000000, "4.0": 0x40800000, "-4.0": 0xC0800000}
        if tok in fl:
            return fl[tok]
        if tok.startswith("0x"):
            return int(tok, 16)
        return int(tok)

    @staticmethod
    def mask_int(m):
        return int(np.packbits(m[::-1].astype(np.uint8)).view(">u8")[0]) if m.size == 64 else 0

    @staticmethod
    def int_mask(x):
        return np.array([(x >> i) & 1 for i in range(64)], bool)

    def check_pending(self, w, kind, base, n):
        for i in range(base, base + n):
            if w.pending_regs.get((kind, i), 0):
                raise EmuError(f"wave {w.wid} pc {w.pc} reads {kind}{i} with a load in flight: {self.ins[w.pc][2]}")

    def rd_v(self, w, tok, n=1):
        """vector source -> uint32 array [n, 64] (or broadcast scalar)"""
        r = reg_range(tok)
        if r and r[0] in "va":
            k, i, cnt = r
            self.check_pending(w, k, i, cnt)
            arr = w.v if k == "v" else w.a
            return arr[i:i + cnt].copy()
        val = self.rd_s(w, tok)
        return np.full((n, 64), val & 0xFFFFFFFF, np.uint32)

    def wr_v(self, w, tok, vals, mask=None):
        k, i, cnt = reg_range(tok)
        arr = w.v if k == "v" else w.a
        vals = np.asarray(vals, np.uint32).reshape(cnt, 64)
        m = w.exec if mask is None else mask
        if w.pending_regs:
            for j in range(i, i + cnt):
                if w.pending_regs.get((k, j), 0):
                    raise EmuError(f"wave {w.wid} pc {w.pc} writes {k}{j} with a load in flight")
        arr[i:i + cnt, m] = vals[:, m]

    def wr_s(self, w, tok, val):
        if tok == "m0":
            w.m0 = val & 0xFFFFFFFF
            return
        if tok == "vcc":
            w.vcc = self.int_mask(val)
            return
        if tok == "exec":
            w.exec = self.int_mask(val)
            return
        k, i, n = reg_range(tok)
        assert k == "s"
        w.s[i] = val & 0xFFFFFFFF
        if n == 2:
            w.s[i + 1] = (val >> 32) & 0xFFFFFFFF

    # ---- async
    def retire_lgkm(self, w, keep):
        while len(w.lgkm) > keep:
            k, base, vals = w.lgkm.pop(0)
            for j in range(vals.shape[0]):
                w.pending_regs[(k, base + j)] -= 1
            arr = w.v if k == "v" else w.a
            arr[base:base + vals.shape[0]] = vals

    def retire_vm(self, w, keep):
        while len(w.vm) > keep:
            item = w.vm.pop(0)
            if item[0] == "reg":
                _, k, base, vals, mask = item
                for j in range(vals.shape[0]):
                    w.pending_regs[(k, base + j)] -= 1
                arr = w.v if k == "v" else w.a
                arr[base:base + vals.shape[0], mask] = vals[:, mask]
            elif item[0] == "lds":
                _, addr, data = item
                self.lds[addr:addr + len(data)] = data
                self.lds_pending[addr:addr + len(data)] -= 1
            # stores complete immediately (written at issue)

    def lds_read(self, w, addr, n):
        if addr < 0 or addr + n > len(self.lds):
            raise EmuError(f"wave {w.wid} pc {w.pc}: LDS read out of range {addr}")
        if self.lds_pending[addr:addr + n].any():
            raise EmuError(f"wave {w.wid} pc {w.pc}: LDS read of bytes with a DMA in flight at {addr}: {self.ins[w.pc][2]}")
        return self.lds[addr:addr + n]

    # ---- run
    def run(self):
        steps = 0
        while True:
            live = [w for w in self.waves if not w.done]
            if not live:
                return
            progressed = False
            for w in live:
                while not w.done and not w.at_barrier:
                    self.step(w)
                    steps += 1
                    progressed = True
                    if steps > self.max_steps:
                        raise EmuError("step limit (infinite loop?)")
            live = [w for w in self.waves if not w.done]
            if live and all(w.at_barrier for w in live):
                if any(w.done for w in self.waves):
                    raise EmuError("barrier reached while another wave has ended")
                for w in live:
                    w.at_barrier = False
                    w.pc += 1
            elif not progressed:
                raise EmuError("deadlock")

    def step(self, w):
        if w.pc >= len(self.ins):
            w.done = True
            return
        op, args, text = self.ins[w.pc]
        self.trace_counts[op] = self.trace_counts.get(op, 0) + 1
        w.count += 1
        fn = getattr(self, "op_" + op, None)
        if fn is None:
            raise EmuError(f"unsupported op {op}: {text}")
        jump = fn(w, args)
        if jump is None:
            w.pc += 1
        elif jump == "barrier":
            w.at_barrier = True
        else:
            w.pc = jump

    # ---- scalar ops
    def op_s_nop(self, w, a): pass

    def op_s_waitcnt(self, w, a):
        txt = " ".join(a)
        m = re.search(r"vmcnt\((\d+)\)", txt)
        if m:
            self.retire_vm(w, int(m.group(1)))
        m = re.search(r"lgkmcnt\((\d+)\)", txt)
        if m:
            self.retire_lgkm(w, int(m.group(1)))

    def op_s_barrier(self, w, a):
        return "barrier"

    def op_s_mov_b32(self, w, a):
        self.wr_s(w, a[0], self.rd_s(w, a[1]))

    def op_s_mov_b64(self, w, a):
        self.wr_s(w, a[0], self.rd_s(w, a[1]))

    def op_s_add_u32(self, w, a):
        x = self.rd_s(w, a[1]) + (self.label_expr(a[2]) if "-" in a[2] and not a[2].startswith("-") else self.rd_s(w, a[2]))
        w.scc = int(x >> 32 & 1)
        self.wr_s(w, a[0], x & 0xFFFFFFFF)

    def label_expr(self, e):
        l, r = [t.strip() for t in e.split(" - ")]
        return (self.labels[l] - self.labels[r]) * 8

    def op_s_addc_u32(self, w, a):
        x = self.rd_s(w, a[1]) + self.rd_s(w, a[2]) + w.scc
        w.scc = int(x >> 32 & 1)
        self.wr_s(w, a[0], x & 0xFFFFFFFF)

    def op_s_sub_u32(self, w, a):
        x = (self.rd_s(w, a[1]) - self.rd_s(w, a[2]))
        w.scc = int(x < 0)
        self.wr_s(w, a[0], x & 0xFFFFFFFF)

    def op_s_lshl_b32(self, w, a):
        x = (self.rd_s(w, a[1]) << self.rd_s(w, a[2])) & 0xFFFFFFFF
        w.scc = int(x != 0)
        self.wr_s(w, a[0], x)

    def op_s_cmp_eq_u32(self, w, a):
        w.scc = int(self.rd_s(w, a[0]) == self.rd_s(w, a[1]))

    def op_s_cmp_lt_u32(self, w, a):
        w.scc = int(self.rd_s(w, a[0]) < self.rd_s(w, a[1]))

    def op_s_cmp_eq_u64(self, w, a):
        w.scc = int(self.rd_s(w, a[0]) == self.rd_s(w, a[1]))

    def op_s_bitcmp1_b32(self, w, a):
        w.scc = int((self.rd_s(w, a[0]) >> self.rd_s(w, a[1])) & 1)

    def op_s_cselect_b32(self, w, a):
        self.wr_s(w, a[0], self.rd_s(w, a[1]) if w.scc else self.rd_s(w, a[2]))

    def op_s_or_b64(self, w, a):
        x = self.rd_s(w, a[1]) | self.rd_s(w, a[2])
        w.scc = int(x != 0)
        self.wr_s(w, a[0], x)

    def op_s_and_b64(self, w, a):
        x = self.rd_s(w, a[1]) & self.rd_s(w, a[2])
        w.scc = int(x != 0)
        self.wr_s(w, a[0], x)

    def op_s_and_saveexec_b64(self, w, a):
        old = self.mask_int(w.exec)
        self.wr_s(w, a[0], old)
        x = old & self.rd_s(w, a[1])
        w.exec = self.int_mask(x)
        w.scc = int(x != 0)

    def op_s_branch(self, w, a):
        return self.labels[a[0]]

    def op_s_cbranch_scc0(self, w, a):
        return self.labels[a[0]] if w.scc == 0 else None

    def op_s_cbranch_scc1(self, w, a):
        return self.labels[a[0]] if w.scc == 1 else None

    def op_s_cbranch_vccz(self, w, a):
        return self.labels[a[0]] if not w.vcc.any() else None

    def op_s_getpc_b64(self, w, a):
        self.wr_s(w, a[0], (w.pc + 1) * 8)

    def op_s_swappc_b64(self, w, a):
        tgt = self.rd_s(w, a[1])
        self.wr_s(w, a[0], (w.pc + 1) * 8)
        assert tgt % 8 == 0
        return tgt // 8

    def op_s_setpc_b64(self, w, a):
        tgt = self.rd_s(w, a[0])
        return tgt // 8

    # ---- VALU
    def fv(self, w, tok):
        return f32(self.rd_v(w, tok)[0])

    def iv(self, w, tok):
        return self.rd_v(w, tok)[0].astype(np.int64)

    def wf(self, w, tok, x):
        self.wr_v(w, tok, u32(np.asarray(x, np.float32)).reshape(1, 64))

    def wi(self, w, tok, x):
        self.wr_v(w, tok, (np.asarray(x, np.int64) & 0xFFFFFFFF).astype(np.uint32).reshape(1, 64))

    def op_v_mov_b32(self, w, a): self.wr_v(w, a[0], self.rd_v(w, a[1]))
    op_v_mov_b32_e32 = op_v_mov_b32
    def op_v_and_b32(self, w, a): self.wi(w, a[0], self.iv(w, a[1]) & self.iv(w, a[2]))
    def op_v_or_b32(self, w, a): self.wi(w, a[0], self.iv(w, a[1]) | self.iv(w, a[2]))
    def op_v_xor_b32(self, w, a): self.wi(w, a[0], self.iv(w, a[1]) ^ self.iv(w, a[2]))
    def op_v_lshrrev_b32(self, w, a): self.wi(w, a[0], self.iv(w, a[2]) >> (self.iv(w, a[1]) & 31))
    def op_v_lshlrev_b32(self, w, a): self.wi(w, a[0], self.iv(w, a[2]) << (self.iv(w, a[1]) & 31))
    def op_v_add_u32(self, w, a): self.wi(w, a[0], self.iv(w, a[1]) + self.iv(w, a[2]))
    def op_v_add3_u32(self, w, a): self.wi(w, a[0], self.iv(w, a[1]) + self.iv(w, a[2]) + self.iv(w, a[3]))
    def op_v_lshl_add_u32(self, w, a): self.wi(w, a[0], (self.iv(w, a[1]) << self.iv(w, a[2])) + self.iv(w, a[3]))
    def op_v_mul_lo_u32(self, w, a): self.wi(w, a[0], self.iv(w, a[1]) * self.iv(w, a[2]))
    def op_v_min_u32(self, w, a): self.wi(w, a[0], np.minimum(self.iv(w, a[1]), self.iv(w, a[2])))
    def op_v_bfe_u32(self, w, a):
        x, o, n = self.iv(w, a[1]), self.iv(w, a[2]), self.iv(w, a[3])
        self.wi(w, a[0], (x >> o) & ((1 << n) - 1))

    def op_v_readfirstlane_b32(self, w, a):
        v = self.rd_v(w, a[1])[0]
        first = int(np.argmax(w.exec))
        self.wr_s(w, a[0], int(v[first]))

    def op_v_fma_f32(self, w, a):
        x, y, z = (self.fv(w, t).astype(np.float64) for t in a[1:4])
        self.wf(w, a[0], (x * y + z).astype(np.float32))

    def op_v_mul_f32(self, w, a): self.wf(w, a[0], self.fv(w, a[1]) * self.fv(w, a[2]))
    def op_v_add_f32(self, w, a): self.wf(w, a[0], self.fv(w, a[1]) + self.fv(w, a[2]))
    def op_v_sub_f32(self, w, a): self.wf(w, a[0], self.fv(w, a[1]) - self.fv(w, a[2]))
    def op_v_max_f32(self, w, a): self.wf(w, a[0], np.fmax(self.fv(w, a[1]), self.fv(w, a[2])))
    def op_v_max3_f32(self, w, a): self.wf(w, a[0], np.fmax(np.fmax(self.fv(w, a[1]), self.fv(w, a[2])), self.fv(w, a[3])))
    def op_v_exp_f32(self, w, a):
        with np.errstate(over="ignore", invalid="ignore"):
            self.wf(w, a[0], np.exp2(self.fv(w, a[1]).astype(np.float64)).astype(np.float32))
    def op_v_log_f32(self, w, a):
        with np.errstate(divide="ignore", invalid="ignore"):
            self.wf(w, a[0], np.log2(self.fv(w, a[1]).astype(np.float64)).astype(np.float32))
    def op_v_rcp_f32(self, w, a):
        with np.errstate(divide="ignore"):
            self.wf(w, a[0], (1.0 / self.fv(w, a[1]).astype(np.float64)).astype(np.float32))

    def op_v_cvt_pk_f16_f32(self, w, a):
        lo = self.fv(w, a[1]).astype(F16).view(np.uint16).astype(np.uint32)
        hi = self.fv(w, a[2]).astype(F16).view(np.uint16).astype(np.uint32)
        self.wr_v(w, a[0], (lo | (hi << 16)).reshape(1, 64))

    def op_v_dot2_f32_f16(self, w, a):
        x = self.rd_v(w, a[1])[0]
        y = self.rd_v(w, a[2])[0]
        z = self.fv(w, a[3]).astype(np.float64)
        xl = (x & 0xFFFF).astype(np.uint16).view(F16).astype(np.float64)
        xh = (x >> 16).astype(np.uint16).view(F16).astype(np.float64)
        yl = (y & 0xFFFF).astype(np.uint16).view(F16).astype(np.float64)
        yh = (y >> 16).astype(np.uint16).view(F16).astype(np.float64)
        self.wf(w, a[0], (xl * yl + xh * yh + z).astype(np.float32))

    def cmp(self, w, a, fn, ints=False):
        x = self.iv(w, a[1]) if ints else self.fv(w, a[1])
        y = self.iv(w, a[2]) if ints else self.fv(w, a[2])
        with np.errstate(invalid="ignore"):
            res = fn(x, y) & w.exec
        if a[0] == "vcc":
            w.vcc = res
        else:
            self.wr_s(w, a[0], self.mask_int(res))

    def op_v_cmp_lt_f32(self, w, a): self.cmp(w, a, np.less)
    op_v_cmp_lt_f32_e64 = op_v_cmp_lt_f32
    def op_v_cmp_le_f32(self, w, a): self.cmp(w, a, np.less_equal)
    def op_v_cmp_eq_f32(self, w, a): self.cmp(w, a, np.equal)
    def op_v_cmp_gt_u32(self, w, a): self.cmp(w, a, np.greater, True)
    def op_v_cmp_eq_u32(self, w, a): self.cmp(w, a, np.equal, True)

    def op_v_cndmask_b32(self, w, a):
        m = w.vcc if a[3] == "vcc" else self.int_mask(self.rd_s(w, a[3]))
        x, y = self.rd_v(w, a[1])[0], self.rd_v(w, a[2])[0]
        self.wr_v(w, a[0], np.where(m, y, x).reshape(1, 64))
    op_v_cndmask_b32_e64 = op_v_cndmask_b32

    def op_v_permlane32_swap_b32(self, w, a):
        x, y = self.rd_v(w, a[0])[0].copy(), self.rd_v(w, a[1])[0].copy()
        nx, ny = x.copy(), y.copy()
        nx[32:] = y[:32]
        ny[:32] = x[32:]
        self.wr_v(w, a[0], nx.reshape(1, 64))
        self.wr_v(w, a[1], ny.reshape(1, 64))

    def op_v_accvgpr_read_b32(self, w, a): self.wr_v(w, a[0], self.rd_v(w, a[1]))
    def op_v_accvgpr_write_b32(self, w, a): self.wr_v(w, a[0], self.rd_v(w, a[1]))
    def op_v_accvgpr_mov_b32(self, w, a): self.wr_v(w, a[0], self.rd_v(w, a[1]))

    def op_v_mfma_f32_32x32x16_f16(self, w, a):
        A = self.rd_v(w, a[1], 4)  # 4 regs x 64 lanes: 8 halves per lane
        B = self.rd_v(w, a[2], 4)
        Cr = a[3]
        if Cr == "0":
            C = np.zeros((16, 64), np.float32)
        else:
            C = f32(self.rd_v(w, Cr, 16))
        ah = A.T.copy().view(np.uint16).view(F16).astype(np.float64).reshape(64, 8)  # lane, k-slot
        bh = B.T.copy().view(np.uint16).view(F16).astype(np.float64).reshape(64, 8)
        Am = np.zeros((32, 16))
        Bm = np.zeros((16, 32))
        for l in range(64):
            Am[l % 32, 8 * (l // 32):8 * (l // 32) + 8] = ah[l]
            Bm[8 * (l // 32):8 * (l // 32) + 8, l % 32] = bh[l]
        Cm = np.zeros((32, 32))
        for l in range(64):
            for i in range(16):
                Cm[8 * (i // 4) + 4 * (l // 32) + i % 4, l % 32] = C[i, l]
        Dm = (Am @ Bm + Cm).astype(np.float32)
        D = np.zeros((16, 64), np.float32)
        for l in range(64):
            for i in range(16):
                D[i, l] = Dm[8 * (i // 4) + 4 * (l // 32) + i % 4, l % 32]
        self.wr_v(w, a[0], u32(D), mask=np.ones(64, bool))

    # ---- memory
    def ds_addr(self, w, a):
        base = self.rd_v(w, a[1])[0].astype(np.int64)
        off = 0
        for t in a[2:]:
            m = re.match(r"offset:(\d+)", t)
            if m:
                off = int(m.group(1))
        if len(a) > 1 and " offset:" in a[1]:
            pass
        return base + off

    def split_off(self, a):
        # 'v8 offset:8192' arrives as one token
        out = []
        off = 0
        for t in a:
            m = re.match(r"(.*?)\s+offset:(\d+)$", t)
            if m:
                out.append(m.group(1))
                off = int(m.group(2))
            else:
                out.append(t)
        return out, off

    def op_ds_read_b128(self, w, a):
        a, off = self.split_off(a)
        addr = self.rd_v(w, a[1])[0].astype(np.int64) + off
        k, base, n = reg_range(a[0])
        vals = np.zeros((4, 64), np.uint32)
        for l in range(64):
            if w.exec[l]:
                vals[:, l] = self.lds_read(w, int(addr[l]), 16).view(np.uint32)
        self.push_lgkm(w, k, base, vals)

    def op_ds_read_b64_tr_b16(self, w, a):
        a, off = self.split_off(a)
        addr = self.rd_v(w, a[1])[0].astype(np.int64) + off
        k, base, n = reg_range(a[0])
        vals = np.zeros((2, 64), np.uint32)
        for g in range(4):
            for j in range(16):
                halves = []
                for h in range(4):
                    src_lane = 16 * g + 4 * h + j // 4
                    p = int(addr[src_lane]) + 2 * (j % 4)
                    halves.append(int(self.lds_read(w, p, 2).view(np.uint16)[0]))
                vals[0, 16 * g + j] = halves[0] | (halves[1] << 16)
                vals[1, 16 * g + j] = halves[2] | (halves[3] << 16)
        self.push_lgkm(w, k, base, vals)

    def push_lgkm(self, w, k, base, vals):
        for j in range(vals.shape[0]):
            w.pending_regs[(k, base + j)] = w.pending_regs.get((k, base + j), 0) + 1
        w.lgkm.append((k, base, vals))
        if len(w.lgkm) > 15:
            raise EmuError(f"wave {w.wid} pc {w.pc}: more than 15 LDS reads outstanding")

    def glob(self, w, a):
        a, off = self.split_off(a)
        return a, off

    def op_global_load_lds_dwordx4(self, w, a):
        a, off = self.split_off(a)
        voff = self.rd_v(w, a[0])[0].astype(np.int64)
        sbase = self.rd_s(w, a[1])
        for l in range(64):
            if not w.exec[l]:
                continue
            data = self.mem.read(sbase + int(voff[l]) + off, 16).copy()
            dst = w.m0 + 16 * l
            if dst < 0 or dst + 16 > len(self.lds):
                raise EmuError(f"wave {w.wid} pc {w.pc}: DMA to LDS out of range {dst}")
            self.lds_pending[dst:dst + 16] += 1
            w.vm.append(("lds", dst, data))
        if len(w.vm) > 64 * 63:
            raise EmuError("vmcnt overflow")

    def op_global_load_dwordx4(self, w, a):
        a, off = self.split_off(a)
        voff = self.rd_v(w, a[1])[0].astype(np.int64)
        sbase = self.rd_s(w, a[2])
        k, base, n = reg_range(a[0])
        vals = np.zeros((4, 64), np.uint32)
        for l in range(64):
            if w.exec[l]:
                vals[:, l] = self.mem.read(sbase + int(voff[l]) + off, 16).view(np.uint32)
        for j in range(4):
            w.pending_regs[(k, base + j)] = w.pending_regs.get((k, base + j), 0) + 1
        w.vm.append(("reg", k, base, vals, w.exec.copy()))

    def store(self, w, a, nregs):
        a, off = self.split_off(a)
        voff = self.rd_v(w, a[0])[0].astype(np.int64)
        data = self.rd_v(w, a[1], nregs)
        sbase = self.rd_s(w, a[2])
        for l in range(64):
            if w.exec[l]:
                self.mem.write(sbase + int(voff[l]) + off, data[:, l].copy().view(np.uint8))
        w.vm.append(("store",))

    def op_global_store_dwordx2(self, w, a): self.store(w, a, 2)
    def op_global_store_dword(self, w, a): self.store(w, a, 1)
