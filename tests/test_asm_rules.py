"""Wait states that inline assembly in the kernels must carry itself (CPU).

The compiler inserts the hazard wait states its own instructions need, but it
does not look inside an `asm` block. A vector memory instruction that reads
SGPRs (a buffer resource, or M0 as the LDS base of an LDS DMA) needs five wait
states after a VALU write of those SGPRs (v_readfirstlane) or after the write
of M0. Without them the load can use a stale base address: the first
software-pipelined DiT build faulted the GPU exactly so. Every inline-asm
memory instruction of csrc/ that takes SGPR or M0 operands must therefore
start its block with `s_nop N`, N >= 4 (N + 1 wait states), or name its wait
in a comment `// wait-states: <reason>` on the line before the `asm`."""
import os
import re

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "pega-omni_amd", "csrc")
VMEM = re.compile(r"(buffer_|global_|flat_|scratch_)(load|store|atomic)")
SNOP = re.compile(r'^\s*"\s*s_nop\s+(\d+)')


def asm_blocks(text):
    """(line, template, operands, preceding line) for every asm statement."""
    out = []
    for m in re.finditer(r"asm\s+(?:volatile\s*)?\(", text):
        depth, i = 1, m.end()
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        body = text[m.end():i - 1]
        parts = body.split(":", 1)
        line = text.count("\n", 0, m.start()) + 1
        prev = text[:m.start()].rstrip().rsplit("\n", 1)[-1]
        out.append((line, parts[0], parts[1] if len(parts) > 1 else "", prev))
    return out


def sources():
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".cpp", ".h")):
            yield f, open(os.path.join(CSRC, f)).read()


def test_asm_memory_ops_reading_sgprs_carry_their_wait_states():
    checked = 0
    for name, text in sources():
        for line, template, operands, prev in asm_blocks(text):
            if not VMEM.search(template):
                continue
            reads_sgpr = re.search(r'"s"|"\{m0\}"|\bm0\b', operands + template) is not None
            if not reads_sgpr:
                continue
            checked += 1
            nop = SNOP.match(template)
            stated = "wait-states:" in prev
            assert stated or (nop and int(nop.group(1)) >= 4), (
                f"{name}:{line}: inline-asm memory instruction reads SGPRs/M0 without a leading s_nop >= 4")
    assert checked >= 2  # the two LDS DMA helpers of tiled.hip


def test_the_lds_dma_helpers_keep_their_s_nop():
    text = open(os.path.join(CSRC, "tiled.hip")).read()
    for fn in ("dma_buffer16", "dma_global16"):
        m = re.search(fn + r"\([^)]*\)\s*\{(.*?)\n\}", text, flags=re.S)
        assert m, fn
        assert re.search(r'asm volatile\("s_nop 4\\n\\t', m.group(1)), f"{fn} lost its leading s_nop 4"


def test_the_checker_catches_a_missing_wait():
    bad = 'asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(x), "s"(r), "{m0}"(l) : "memory");'
    (line, template, operands, prev), = asm_blocks(bad)
    assert VMEM.search(template) and re.search(r'"s"', operands) and not SNOP.match(template)
