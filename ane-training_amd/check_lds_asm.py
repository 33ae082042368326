"""Build check of k_gemm.hip's inline LDS reads (run by `make check`).

The tiled GEMM issues its fragment reads (ds_read_b128) as inline assembly and
waits for them with a separate `s_waitcnt lgkmcnt(0)` statement that names the
destination registers as in/out operands.  The compiler cannot see that a read
is still in flight between the two statements; this script scans the device
assembly of every k_gemm_tile instantiation and fails if any instruction
reads or writes the destination register of an LDS read that no wait has
retired yet: lgkmcnt(0) retires every read, and the compiler's own
lgkmcnt(n) retires all but the n youngest LDS operations when no scalar load
is in flight (LDS operations complete in order).

    python3 check_lds_asm.py k_gemm.s
"""
import re
import sys


def regset(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {tok} if m else set()


def check(asm_text):
    bad = []
    names = re.findall(r"^(_Z11k_gemm_tile\S*):", asm_text, re.M)
    for name in names:
        a = asm_text.index(name + ":")
        b = asm_text.index(".Lfunc_end", a)
        # lgkm operations in flight, oldest first: (destination registers, is
        # scalar memory).  LDS operations complete in order, so a wait
        # lgkmcnt(n) retires all but the n youngest; scalar loads complete out
        # of order, so with one in flight only lgkmcnt(0) retires anything.
        queue = []
        for ln in asm_text[a:b].split("\n"):
            t = ln.split(";")[0].strip()
            if not t or t.startswith("."):
                continue
            ops = [x for x in re.split(r"[ ,]+", t) if x]
            if ops[0].startswith("ds_"):
                dst = regset(ops[1]) if ops[0].startswith(("ds_read", "ds_bpermute", "ds_permute",
                                                           "ds_swizzle")) else set()
                queue.append((dst, False))
                continue
            if ops[0].startswith(("s_load", "s_buffer_load")):
                queue.append((set(), True))
                continue
            if ops[0] == "s_waitcnt":
                m = re.search(r"lgkmcnt\((\d+)\)", t)
                if m:
                    n = int(m.group(1))
                    if n == 0:
                        queue = []
                    elif not any(s for _, s in queue):
                        queue = queue[-n:] if n < len(queue) else queue
                continue
            pending = set().union(*(d for d, _ in queue)) if queue else set()
            if pending:
                used = set()
                for o in ops[1:]:
                    used |= regset(o)
                if used & pending:
                    bad.append((name, t))
    return names, bad


def main():
    names, bad = check(open(sys.argv[1]).read())
    if not names:
        print("check_lds_asm: no k_gemm_tile functions found", file=sys.stderr)
        return 1
    for name, t in bad:
        print(f"check_lds_asm: {name}: pending LDS read register used by: {t}", file=sys.stderr)
    if bad:
        return 1
    print(f"check_lds_asm: {len(names)} tile kernels, no use of a pending LDS read")
    return 0


if __name__ == "__main__":
    sys.exit(main())
