"""Source-level rules for the gfx950 kernels (flash_fwd.hip), checked on the CPU.

Every load that writes registers must be one the compiler issues, or must wait for its own result
in the same asm statement. An asm statement that issues a load into output registers and returns
before the data has landed leaves the compiler holding registers it believes valid: any copy,
spill or reuse it places before the separate wait reads or clobbers data in flight, with no
diagnostic. The buffer->LDS loads (`... lds`) write no registers and are waited for explicitly.
"""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNEL_SOURCES = [os.path.join(ROOT, "not-cute-zig_amd", "csrc", f) for f in ("flash_fwd.hip", "hw_probe.hip")]

LOAD = re.compile(r"\b(buffer_load|global_load|flat_load|scratch_load|ds_read|ds_load|s_load|s_buffer_load)\w*")


def asm_statements(src):
    """(template text, output operand list) of every asm statement."""
    out = []
    for m in re.finditer(r"\basm\s+(?:volatile\s*)?\(", src):
        depth, i = 1, m.end()
        while depth:
            c = src[i]
            if c == '"':
                i = src.index('"', i + 1)
                while src[i - 1] == "\\":
                    i = src.index('"', i + 1)
            elif c == "(":
                depth += 1
            elif c == ")":
                depth -= 1
            i += 1
        body = src[m.end():i - 1]
        # the template's string literals come first; operand lists follow the first ':' outside them
        literals = re.compile(r'\s*"((?:[^"\\]|\\.)*)"')
        pos, parts = 0, []
        while (lit := literals.match(body, pos)):
            parts.append(lit.group(1))
            pos = lit.end()
        rest = body[pos:].lstrip()
        outputs = "" if rest.startswith("::") or not rest.startswith(":") else rest[1:].split(":")[0]
        out.append(("".join(parts), outputs))
    return out


def window_loads(src):
    bad = []
    for template, outputs in asm_statements(src):
        writes = '"=' in outputs or '"+' in outputs
        for line in template.split("\\n"):
            if LOAD.search(line) and not re.search(r"\blds\b", line) and writes and "s_waitcnt" not in template:
                bad.append(template)
    return bad


def test_no_asm_load_returns_before_its_data():
    for path in KERNEL_SOURCES:
        with open(path) as f:
            src = f.read()
        assert window_loads(src) == [], path


def test_rule_catches_a_planted_window():
    """The checker itself: an asm load with an output and no wait is flagged; the same load with
    its wait in the statement, a buffer->LDS load, and a store are not."""
    planted = 'asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(out) : "v"(addr));'
    assert window_loads(planted)
    planted_q = 'asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(dst) : "v"(o), "s"(r));'
    assert window_loads(planted_q)
    assert not window_loads('asm volatile("global_load_dwordx4 %0, %1, off\\n\\ts_waitcnt vmcnt(0)" : "=&v"(x) : "v"(p));')
    assert not window_loads('asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" :: "v"(o), "s"(r));')
    assert not window_loads('asm volatile("global_store_dwordx4 %0, %1, off" ::"v"(p), "v"(v) : "memory");')
