"""Build check of k_gemm.hip's inline LDS reads (run by `make check`).

The tiled GEMM issues its fragment reads (ds_read_b128) as inline assembly and
waits for them with a separate `s_waitcnt lgkmcnt(0)` statement that names the
destination registers as in/out operands.  The compiler cannot see that a read
is still in flight between the two statements; this script scans the device
assembly of every k_gemm_tile instantiation and fails if any instruction
between a read and the next lgkmcnt(0) wait reads or writes one of the pending
destination registers.

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
        pending = set()
        for ln in asm_text[a:b].split("\n"):
            t = ln.split(";")[0].strip()
            if not t or t.startswith("."):
                continue
            ops = [x for x in re.split(r"[ ,]+", t) if x]
            if ops[0] == "ds_read_b128":
                pending |= regset(ops[1])
                continue
            if ops[0] == "s_waitcnt" and "lgkmcnt(0)" in t:
                pending = set()
                continue
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
