"""Source rules of the HIP kernels (CPU only, reads qengine_amd/csrc).

* No VALU instruction in inline asm. The compiler inserts the wait states that gfx950 needs between an MFMA and a
  vector instruction that reads its result or overwrites a register the MFMA still reads (srcC) or writes, but its
  hazard checks do not look into inline asm operands: a `v_...` asm statement scheduled close behind an MFMA can
  overwrite srcC while the MFMA is still reading it, which corrupts the product silently. Scalar moves, LDS DMA,
  waits and barriers in asm are allowed.
* Every asm LDS DMA (global_load_lds_*) is preceded in its statement by the scalar write of m0 and one s_nop: on
  GFX9 an LDS DMA needs one wait state after a scalar write of m0, which the compiler cannot insert into asm.
* No __builtin_bit_cast whose operand is a subscripted element (`__builtin_bit_cast(int, v[r])`): this hipcc lowers
  the bit_cast of an ext_vector_type element as a load of the vector's first element, whatever the index (seen on
  gfx950 with ROCm 7.2: every lane of an unrolled loop got element 0). Copy the element into a scalar first.
"""
import os
import re

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qengine_amd", "csrc")


def asm_statements():
    for f in sorted(os.listdir(CSRC)):
        if not f.endswith((".hip", ".hpp", ".cpp")):
            continue
        txt = open(os.path.join(CSRC, f)).read()
        txt = re.sub(r"//[^\n]*", "", txt)
        for m in re.finditer(r"\basm\s*(?:volatile\s*)?\(\s*((?:\"(?:[^\"\\]|\\.)*\"\s*)+)", txt):
            body = "".join(re.findall(r"\"((?:[^\"\\]|\\.)*)\"", m.group(1)))
            yield f, body.replace("\\n", "\n").replace("\\t", " ")


def test_asm_statements_found():
    assert any("global_load_lds" in b for _, b in asm_statements())


def test_no_valu_inline_asm():
    bad = [(f, b) for f, b in asm_statements() if re.search(r"(^|\s)v_[a-z0-9_]+", b)]
    assert not bad, bad


def test_lds_dma_asm_waits_after_m0():
    for f, b in asm_statements():
        ins = [l.strip().split()[0] for l in b.split("\n") if l.strip()]
        for i, op in enumerate(ins):
            if op.startswith("global_load_lds"):
                assert i >= 2 and ins[i - 1] == "s_nop" and ins[i - 2] == "s_mov_b32", (f, b)


def test_no_bit_cast_of_subscripted_element():
    bad = []
    for f in sorted(os.listdir(CSRC)):
        if not f.endswith((".hip", ".hpp", ".cpp")):
            continue
        txt = re.sub(r"//[^\n]*", "", open(os.path.join(CSRC, f)).read())
        for m in re.finditer(r"__builtin_bit_cast\(\s*[^,()]+,\s*[A-Za-z_][A-Za-z0-9_.]*(\[[^\]]+\])+\s*\)", txt):
            bad.append((f, m.group(0)))
    assert not bad, bad
