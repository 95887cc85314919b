"""Build-time check of k_mx_mfma's inline-assembly weight loads.

The grouped GEMV issues each row tile's loads with inline assembly and waits
for them with one `s_waitcnt vmcnt(0)` at the top of the next step (marked
with the comment `spt tile wait` in the assembly); the
compiler does not know that the load registers are written asynchronously.
This scans the gfx950 assembly of spt_mx_mfma.hip (hipcc -S) and fails if any
instruction other than the loads, that wait and the LDS stores that consume
the registers reads or writes a load register between the issue and the
wait: a copy, spill or reuse there would see stale data.

Usage: python3 isa_check.py <assembly.s>
"""
import re
import sys


def vregs(text):
    out = set()
    for a, b in re.findall(r'\bv\[(\d+):(\d+)\]', text):
        out |= set(range(int(a), int(b) + 1))
    for a in re.findall(r'\bv(\d+)\b', text):
        out.add(int(a))
    return out


def check_kernel(lines):
    ins = [(k, l.split(';')[0].strip()) for k, l in enumerate(lines)]
    ins = [(k, l) for k, l in ins if l and not l.endswith(':') and not l.startswith('.')]
    # issue blocks: s_nop 4, then four buffer_load_dwordx4 at offsets 0..3072
    issues = []
    for idx, (k, l) in enumerate(ins):
        if not l.startswith('s_nop 4') or idx + 4 >= len(ins):
            continue
        block = [ins[idx + 1 + q] for q in range(4)]
        if not all(b[1].startswith('buffer_load_dwordx4 v[') for b in block):
            continue
        offs = [re.search(r'offset:(\d+)', b[1]) for b in block]
        if [int(o.group(1)) if o else 0 for o in offs] != [0, 1024, 2048, 3072]:
            continue
        regs = set()
        for b in block:
            regs |= vregs(b[1].split(',')[0])
        issues.append((k, {b[0] for b in block}, regs))
    if not issues:
        return 'no inline-assembly tile loads found'
    tile = set().union(*[r for _, _, r in issues])
    consumers = {k for k, l in ins if l.startswith('ds_write_b128') and vregs(l.split(',', 1)[1]) & tile}
    waits = [k for k, l in enumerate(lines) if 'spt tile wait' in l and l.strip().startswith('s_waitcnt vmcnt(0)')]
    if not waits:
        return 'tile wait not found'
    # the main loop: the outermost loop holding the last tile wait
    loop = None
    for k, l in enumerate(lines):
        if 'Loop Header: Depth=1' not in l or k > waits[-1]:
            continue
        label = l.split(':')[0].strip()
        ends = [j for j, x in ins if re.search(r's_c?branch\w* ' + re.escape(label) + r'$', x)]
        if ends and max(ends) > waits[-1]:
            loop = (k, max(ends))
    if loop is None:
        return 'main loop not found'
    hdr, lend = loop
    last_wait = max(w for w in waits if hdr <= w <= lend) if any(hdr <= w <= lend for w in waits) else None
    if last_wait is None:
        return 'no tile wait in the main loop'
    allowed = consumers.union(*[ks for _, ks, _ in issues]) | set(waits)
    bad = []
    for k0, ks, regs in issues:
        # Conservative windows: from the issue to the loop's end (or, before
        # the loop, to its header), and from the header to the loop's last
        # tile wait, so every path from an issue to the wait that covers it
        # lies inside them.
        windows = [(k0, lend if k0 >= hdr else hdr), (hdr, last_wait)]
        for a, b in windows:
            for k, l in ins:
                if a <= k <= b and k not in allowed and vregs(l) & regs:
                    bad.append('%d: %s' % (k, l))
    return '; '.join(sorted(set(bad))[:5]) if bad else None


def main(path):
    text = open(path).read()
    names = re.findall(r'^(_ZN3spt9k_mx_mfma\w+):', text, re.M)
    if not names:
        print('isa_check: no k_mx_mfma kernels in', path)
        return 1
    failed = 0
    for name in names:
        i = text.index(name + ':')
        j = text.index('.Lfunc_end', i)
        err = check_kernel(text[i:j].split('\n'))
        if err:
            print('isa_check: %s: %s' % (name, err))
            failed = 1
    if not failed:
        print('isa_check: %d kernels, load registers untouched between issue and wait' % len(names))
    return failed


if __name__ == '__main__':
    sys.exit(main(sys.argv[1]))
