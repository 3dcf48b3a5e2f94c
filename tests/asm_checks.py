"""Static checks of the gfx950 assembly of this library's own kernels (test infrastructure).

Several kernels issue MFMAs and vector loads as inline asm, which the compiler schedules around
without seeing inside. Two properties then rest on the code the compiler happens to emit, and
are checked here on the assembly it does emit:

* `mfma_hazards`: no MFMA reads a register (A, B or C operand) that a VALU instruction wrote
  fewer than 2 wait states earlier (the compiler inserts these nops for its own MFMAs only);
* `async_load_touches`: no instruction reads or writes the destination registers of a vector
  load before an `s_waitcnt vmcnt(N)` that covers the load (an inline-asm load's destination is
  written when the data lands, not when the asm statement ends; a register the compiler reuses
  or copies in between is overwritten or read early);
* `lds_load_touches`: the same for LDS reads (`ds_read*`), against the `s_waitcnt lgkmcnt(N)` that
  covers them: several kernels issue fragment reads as inline asm and wait for them with hand-counted
  lgkmcnt values, which rests on the same property. LDS operations complete in issue order, scalar
  memory loads in any order, so a wait covers a read when N is at most the number of LDS
  operations issued after it;
* `mfma_result_touches`: no instruction other than the next MFMA of the same accumulation chain
  (same destination, same C operand) reads or writes an MFMA's destination registers fewer than
  12 wait states after it. 12 is what the compiler itself leaves after its own
  v_mfma_f32_32x32x16_bf16 on gfx950 before reading the result (8 passes + 4); for an inline-asm
  MFMA it leaves nothing, so a spill or copy it places right after one reads stale registers.
  An intervening MFMA counts as 4 wait states (its issue waits for the matrix pipeline, which
  the earlier 8-pass MFMA holds for longer than that).
"""
import re
import subprocess

from noise_amd import build as B


def device_asm(src, tmp_path, defines=()):
    out = tmp_path / (src.stem + '.s')
    cmd = [B.hipcc(), *B.FLAGS, *defines, '--cuda-device-only', '-S', '-x', 'hip', str(src), '-o', str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc -S failed for {src.name}:\n{res.stderr}')
    return out.read_text()


def _regs(tok):
    tok = tok.strip()
    m = re.match(r'([va])\[(\d+):(\d+)\]$', tok)
    if m:
        return {f'{m.group(1)}{i}' for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r'([va])(\d+)$', tok)
    return {tok} if m else set()


def _operands(line):
    parts = line.split(None, 1)
    return [o.strip() for o in re.split(r',(?![^\[]*\])', parts[1])] if len(parts) > 1 else []


def _instructions(asm):
    out = []
    for line in asm.splitlines():
        line = line.split(';')[0].strip()
        if line and not line.startswith('.') and not re.match(r'^\S+:$', line):
            out.append(line)
    return out


def mfma_hazards(asm, need=2):
    ins = _instructions(asm)
    bad = []
    for i, line in enumerate(ins):
        if not line.startswith('v_mfma'):
            continue
        srcs = set().union(*(_regs(o) for o in _operands(line)[1:4]))
        waits = 0
        for j in range(i - 1, max(i - 2 * need - 4, -1), -1):
            prev = ins[j]
            if prev.startswith('v_') and not prev.startswith('v_mfma'):
                ops = _operands(prev)
                if ops and _regs(ops[0]) & srcs and waits < need:
                    bad.append((prev, line))
                    break
            waits += int(prev.split()[1]) + 1 if prev.startswith('s_nop') else 1
            if waits >= need:
                break
    return bad


def mfma_result_touches(asm, need=12, mfma_waits=4):
    ins = _instructions(asm)
    bad = []
    for i, line in enumerate(ins):
        if not line.startswith('v_mfma'):
            continue
        dst = _regs(_operands(line)[0])
        waits = 0
        for nxt in ins[i + 1:]:
            if waits >= need or nxt.startswith(('s_endpgm', 's_branch', 's_setpc')):
                break
            ops = _operands(nxt)
            if nxt.startswith('v_mfma'):
                d2, c2 = _regs(ops[0]), _regs(ops[3])
                ab = _regs(ops[1]) | _regs(ops[2])
                if ab & dst or ((d2 | c2) & dst and not (d2 == dst and c2 == dst)):
                    bad.append((line, nxt))
                    break
                waits += mfma_waits
                continue
            if ops and set().union(*(_regs(o) for o in ops)) & dst:
                bad.append((line, nxt))
                break
            waits += int(nxt.split()[1], 0) + 1 if nxt.startswith('s_nop') else 1
    return bad


def async_load_touches(asm):
    ins = _instructions(asm)
    bad = []
    for i, line in enumerate(ins):
        if not re.match(r'global_load_(dword|dwordx2|dwordx3|dwordx4)\b', line):
            continue
        dst = _regs(_operands(line)[0])
        if not dst:
            continue
        later = 0  # vector memory operations issued after this load
        for nxt in ins[i + 1:]:
            m = re.match(r's_waitcnt\s.*vmcnt\((\d+)\)', nxt)
            if m and int(m.group(1)) <= later:
                break
            if nxt.startswith(('s_endpgm', 's_branch', 's_setpc')):
                break  # conditional branches are scanned through (their fall-through code)
            ops = _operands(nxt)
            if ops and set().union(*(_regs(o) for o in ops)) & dst:
                bad.append((line, nxt))
                break
            if re.match(r'(global_|buffer_|flat_|scratch_)(load|store|atomic)', nxt):
                later += 1
    return bad


def lds_load_touches(asm):
    ins = _instructions(asm)
    bad = []
    for i, line in enumerate(ins):
        if not line.startswith('ds_read'):
            continue
        dst = _regs(_operands(line)[0])
        if not dst:
            continue
        later = 0  # LDS operations issued after this read
        for nxt in ins[i + 1:]:
            m = re.match(r's_waitcnt\s.*lgkmcnt\((\d+)\)', nxt)
            if (m and int(m.group(1)) <= later) or re.match(r's_waitcnt\s+0\s*$', nxt):
                break
            if nxt.startswith(('s_endpgm', 's_branch', 's_setpc')):
                break
            ops = _operands(nxt)
            if ops and set().union(*(_regs(o) for o in ops)) & dst:
                bad.append((line, nxt))
                break
            if nxt.startswith('ds_'):
                later += 1
    return bad


def kernel_spills(asm):
    """{kernel symbol: .vgpr_spill_count} from the code object metadata."""
    names = re.findall(r'\.name:\s+(_Z\S+)', asm)
    spills = [int(v) for v in re.findall(r'\.vgpr_spill_count:\s+(\d+)', asm)]
    return dict(zip(names, spills))


def loop_scratch(asm):
    """(loop headers seen, [(kernel, block, instruction)]): scratch-memory (spill) instructions in
    basic blocks that belong to a loop, as the compiler annotates each block label ('Loop Header',
    'in Loop: Header=...', 'Parent Loop ...')."""
    bad, loops = [], 0
    for m in re.finditer(r'^(_Z\S+):(?:[ \t]*;[^\n]*)?$(.*?)^\.Lfunc_end\d+:', asm, re.M | re.S):
        kernel, body = m.group(1), m.group(2).splitlines()
        in_loop, block = False, 'entry'
        for i, line in enumerate(body):
            lab = re.match(r'^(\.LBB\d+_\d+:|; %bb\.\d+:)', line)
            if lab:
                block = lab.group(1)
                notes = [line] + [body[j] for j in range(i + 1, min(i + 4, len(body)))
                                  if re.match(r'^\s+;', body[j])]
                text = ' '.join(notes)
                in_loop = 'Loop' in text
                loops += 'Loop Header' in text
                continue
            if in_loop and re.match(r'\s*scratch_', line):
                bad.append((kernel, block, line.strip()))
    return loops, bad


def step_barrier_waits(asm):
    """(barriers checked, [(barrier line, wait count, ops after the loads)]), for kernels whose
    stages are loaded one step ahead: every `s_waitcnt vmcnt(N)` that opens an `s_barrier` after
    direct global -> LDS loads (global_load_lds*) must leave only vector memory operations issued
    after the last of those loads in flight, i.e. at least N such operations follow it (they
    retire in order), so that the stage is complete for this wave at the barrier. Scans each
    kernel back to the previous barrier. (A ring loaded two stages ahead, as the fused MLP's
    attention c_proj, waits for the older group on purpose and is not checked this way.)"""
    bad, checked = [], 0
    vmem = re.compile(r'(global_|buffer_|scratch_|flat_)(load|store|atomic)')
    for m in re.finditer(r'^(_Z\S+):(?:[ \t]*;[^\n]*)?$(.*?)^\.Lfunc_end\d+:', asm, re.M | re.S):
        ins = _instructions(m.group(2))
        for i, line in enumerate(ins):
            w = re.match(r's_waitcnt\s.*vmcnt\((\d+)\)', line)
            if not w or not any(x.startswith('s_barrier') for x in ins[i + 1:i + 3]):
                continue
            n, after = int(w.group(1)), 0
            for prev in reversed(ins[:i]):
                if prev.startswith('s_barrier'):
                    break
                if prev.startswith('global_load_lds'):
                    checked += 1
                    if after < n:
                        bad.append((line, n, after))
                    break
                if vmem.match(prev):
                    after += 1
    return checked, bad
