"""The integration guide's error-text lists match the library sources (CPU only).

A Rust binding maps libvtq's VTQ_E_INTERNAL text back onto the reference's
&'static str through the closed list in the integration guide; a text the library
can return but the list lacks would surface as "vtq: internal error".  So
every string literal passed with VTQ_E_INTERNAL in vtq_api.hip must be in
the list, and the list must hold nothing else."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _read(*p):
    with open(os.path.join(ROOT, *p)) as f:
        return f.read()


def library_internal_texts():
    src = _read("vitni-tensor_amd", "csrc", "vtq_api.hip")
    texts = set()
    for m in re.finditer(r"set_err\(c, VTQ_E_INTERNAL,(.*?)\);", src, re.S):
        texts.update(re.findall(r'"([^"]*)"', m.group(1)))
    return texts


def documented_internal_texts():
    doc = _read("INTEGRATION.md")
    block = re.search(r"const INTERNAL_TEXTS: &\[&str\] = &\[(.*?)\];", doc, re.S)
    assert block, "INTERNAL_TEXTS list missing from the integration guide"
    return re.findall(r'"([^"]*)"', block.group(1))


def test_internal_text_list_is_exactly_the_library_set():
    lib = library_internal_texts()
    doc = documented_internal_texts()
    assert len(doc) == len(set(doc)), "duplicate entries"
    assert set(doc) == lib, f"missing: {sorted(lib - set(doc))}; extra: {sorted(set(doc) - lib)}"


def test_reference_texts_are_verbatim():
    """The texts that restate a reference error exist verbatim in the
    reference's arms (checked against the strings it is documented to
    return: every non-"vtq:" entry)."""
    ref = [t for t in documented_internal_texts() if not t.startswith("vtq:")]
    assert len(ref) == 19
    for t in ref:
        assert t.split(":")[0] in ("Q5_0", "Q8_0", "linear_dispatch F32", "linear_dispatch Q5_0",
                                   "linear_dispatch Q8_0", "linear_q4_0", "linear_q4_k_fused",
                                   "linear_q4_k_integer", "linear_q4_k_integer_parallel", "linear_q6_k_integer",
                                   "linear_q6_k_integer_parallel")


def test_runtime_texts_are_documented():
    """Every error text of the GGUF parser and the decode driver appears in
    the integration guide's status table (with {a,b} alternatives expanded)."""
    doc = _read("INTEGRATION.md")
    table = doc[doc.index("| status | `Error` variant |"):]
    table = table[:table.index("All of these checks")]
    expanded = set()
    for cell in re.findall(r"`([^`]+)`", table):
        m = re.search(r"\{([^}]*)\}", cell)
        if not m:
            expanded.add(cell)
            continue
        for alt in m.group(1).split(","):
            expanded.add(cell[:m.start()] + alt.strip() + cell[m.end():])
    src = _read("vitni-tensor_amd", "csrc", "vtq_gguf.cpp") + _read("vitni-tensor_amd", "csrc", "vtq_runtime.hip")
    texts = set(re.findall(r'"((?:gguf: |embedding_row |embedding_row: |prompt|vtq: )[^"]*)"', src))
    texts.discard("prompt_tokens")  # a digest field name, not an error
    missing = set()
    for t in texts:
        if t in expanded:
            continue
        # embedding_row's per-type texts are documented in one braced cell
        if t.startswith("embedding_row ") and t.split(": ", 1)[1] in doc:
            continue
        if t.startswith("vtq: ") and t.split(" (")[0] in doc:
            continue
        missing.add(t)
    assert not missing, sorted(missing)
