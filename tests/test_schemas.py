"""The drop-in boundary: every operator schema the reference registers (the string literals
of its m.def / TORCH_SELECTIVE_SCHEMA / schema_str sites under torchpairwise/csrc) is
registered by this build with the same name, overload, arguments, defaults and returns.
Read from the reference's sources as text; skipped where /root/reference is absent."""
import re
from pathlib import Path

import pytest
import torch

import torchpairwise_amd  # noqa: F401  (registers torch.ops.torchpairwise)

CSRC = Path("/root/reference/torchpairwise/csrc")
pytestmark = pytest.mark.skipif(not CSRC.exists(), reason="reference sources not present")

_SITE = re.compile(r'(?:\bm\.def\s*\(|TORCH_SELECTIVE_SCHEMA\s*\(|\(\s*schema_str\s*,)')


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _pw_tables():
    """op_name's switch tables of common/binary_ops.h:16-43 and common/reduction_ops.h:14-35
    (enum -> name piece) and their signature literal: the pw* schemas are assembled from them
    at run time (pairwise_binary.cpp:135-160, m.def(op_full_schema<Op[, Reduction]>()))."""
    tables, signature = [], None
    for name in ("binary_ops.h", "reduction_ops.h"):
        text = _strip_comments((CSRC / "ops" / "common" / name).read_text())
        tables.append(dict(re.findall(r'case\s+(\w+)\s*:\s*return\s+c10::str\(ns,\s*(?:binary_prefix,\s*)?"(\w+)"', text)))
        m = re.search(r'with_signature\s*\?\s*"([^"]*)"', text)
        signature = signature or (m and m.group(1))
    return tables[0], tables[1], signature


def reference_schemas() -> list[str]:
    """Schema strings (without the namespace) in the order the reference's sources hold them;
    m.def of a bare name (torchpairwise.cpp:54-55) gives the name alone."""
    found = []
    binary, reduction, signature = _pw_tables()
    sources = [p for p in sorted(CSRC.rglob("*")) if p.suffix in (".cpp", ".h")]
    texts = [_strip_comments(p.read_text()) for p in sources]
    # string macros spliced between literals (TORCHPAIRWISE_CPDIST_EXTRA_ARGS_SCHEMA_STR, cpdist.h:7)
    macros = {}
    for text in texts:
        for name, body in re.findall(r'#define\s+(\w+)\s+"((?:[^"\\]|\\.)*)"\s*$', text, flags=re.M):
            macros[name] = body
    piece = re.compile(r'\s*(?:"((?:[^"\\]|\\.)*)"|(' + "|".join(map(re.escape, macros)) + r')\b)')
    for text in texts:
        for op, red in re.findall(r'm\.def\(\s*op_full_schema<\s*(\w+)\s*(?:,\s*(\w+)\s*)?>', text):
            found.append(binary[op] + (f"_{reduction[red]}" if red else "") + signature)
        for site in _SITE.finditer(text):
            pos, parts = site.end(), []
            while (lit := piece.match(text, pos)) is not None:
                raw = lit.group(1) if lit.group(1) is not None else macros[lit.group(2)]
                parts.append(raw.encode().decode("unicode_escape"))
                pos = lit.end()
            s = "".join(parts)
            if not s or s == "torchpairwise::":
                continue
            found.append(s.removeprefix("torchpairwise::"))
    return found


def registered_schemas() -> dict[str, str]:
    out = {}
    for s in torch._C._jit_get_all_schemas():
        if s.name.startswith("torchpairwise::"):
            key = s.name.removeprefix("torchpairwise::") + (f".{s.overload_name}" if s.overload_name else "")
            out[key] = str(s)
    return out


def _key(schema: str) -> str:
    head = schema.split("(", 1)[0]
    return head


def test_every_reference_schema_is_registered_identically():
    ref = reference_schemas()
    assert len(ref) == 101, f"expected the reference's 101 schemas, parsed {len(ref)}"
    ours = registered_schemas()
    missing, different = [], []
    for s in ref:
        if "(" not in s:  # name-only m.def: schema inferred from the C++ function
            inferred = {"_cuda_version": "torchpairwise::_cuda_version() -> int",
                        "_cuda_arch_flags": "torchpairwise::_cuda_arch_flags() -> str"}[s]
            if ours.get(s) != inferred:
                different.append((s, ours.get(s), inferred))
            continue
        want = str(torch._C.parse_schema("torchpairwise::" + s))
        key = _key(s)
        if key not in ours:
            missing.append(key)
        elif ours[key] != want:
            different.append((key, ours[key], want))
    assert not missing, f"not registered: {missing}"
    assert not different, "schemas differ:\n" + "\n".join(f"{k}\n  ours {o}\n  ref  {w}" for k, o, w in different)


def test_schema_parser_reads_known_sites():
    """The extraction sees the three spellings the reference uses."""
    ref = reference_schemas()
    assert 'prf_ldiv_.Scalar(Tensor(a!) input, Scalar other, str mode="zero") -> Tensor(a!)' in ref
    assert "euclidean_distances(Tensor x1, Tensor? x2=None) -> Tensor" in ref
    assert any(s.startswith("cdist(Tensor x1, Tensor x2, str metric=\"minkowski\", *,") for s in ref)
    assert "_cuda_version" in ref
    assert "pwne_mean(Tensor x1, Tensor x2) -> Tensor" in ref and "pwge(Tensor x1, Tensor x2) -> Tensor" in ref
