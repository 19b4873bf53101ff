"""The LDS-DMA kernels' use of M0, checked in the gfx950 code objects of the built libsa3k.so.

The GEMM and attention kernels fill LDS with buffer_load ... lds / global_load_lds, whose LDS
destination comes from the scalar register M0. They issue each one from an inline-asm statement
that writes M0 and the load back to back (csrc/gemm_dma.hip dma16 / dma16b, csrc/attn.hip), so
that the compiler's wait insertion does not drain every DMA before each LDS read; the compiler is
not told that M0 changes. That is correct exactly when no code of the compiler's own keeps a value
in M0 in the same kernel, which this test establishes on the machine code itself, for every
function of the library that issues an LDS DMA:

1. every instruction that names M0 is an `s_mov_b32 m0, ...` immediately followed by an LDS-DMA load;
2. every LDS-DMA load is immediately preceded by such a write (one asm statement, nothing between);
3. no instruction that uses M0 implicitly for another purpose (indexed register access, messages,
   GWS / append / consume / ordered-count LDS operations, interpolation, LDS parameter loads, the
   lane-address LDS operations) appears in it, and it calls no other function.

Functions without LDS DMA run none of these asm statements and may use M0 as the compiler likes
(the adapter-chain fold kernel's indexed register arrays do).

No GPU: the code objects are unbundled from the library and disassembled with the ROCm LLVM tools.
"""
import os
import re
import shutil
import subprocess

import pytest

from conftest import sa3k

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
# instructions that read M0 without naming it
IMPLICIT_M0 = re.compile(r"^(v_movrel|s_movrel|s_sendmsg|ds_gws|ds_append|ds_consume|ds_ordered_count|v_interp|"
                         r"lds_param_load|lds_direct_load|ds_read_addtid|ds_write_addtid|ds_load_addtid|"
                         r"ds_store_addtid|s_set_gpr_idx)")


def _tools():
    need = [os.path.join(LLVM, t) for t in ("clang-offload-bundler", "llvm-objdump")] + [shutil.which("objcopy")]
    missing = [t for t in need if not t or not os.path.exists(t)]
    assert not missing, f"ROCm LLVM tools missing: {missing}"
    return need


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    bundler, objdump, objcopy = _tools()
    d = tmp_path_factory.mktemp("isa")
    fat = d / "fat.bin"
    # objcopy without an output file rewrites its input in place, and this process has the library
    # mapped: dump from a copy, into an explicit output
    lib = d / "lib.so"
    shutil.copyfile(sa3k.LIB_PATH, lib)
    subprocess.run([objcopy, "--dump-section", f".hip_fatbin={fat}", str(lib), str(d / "lib.out")], check=True)
    blob = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), blob)]
    assert starts, "no offload bundles in the library"
    texts = []
    for k, s in enumerate(starts):
        end = starts[k + 1] if k + 1 < len(starts) else len(blob)
        part, co = d / f"b{k}.bundle", d / f"b{k}.co"
        part.write_bytes(blob[s:end])
        subprocess.run([bundler, "--type=o", "--unbundle", f"--input={part}", f"--output={co}", f"--targets={TARGET}"],
                       check=True)
        out = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(co)], check=True, capture_output=True,
                             text=True).stdout
        texts.append(out)
    return texts


def _instructions(text):
    """(mnemonic, operands) per instruction line of an llvm-objdump listing"""
    out = []
    for line in text.splitlines():
        line = line.split("//")[0].strip()
        if not line or line.endswith(":") or line.startswith(("Disassembly", "file format")) or "file format" in line:
            continue
        parts = line.split(None, 1)
        out.append((parts[0], parts[1] if len(parts) > 1 else ""))
    return out


def _is_lds_dma(mn, ops):
    return mn.startswith("global_load_lds_") or (mn.startswith("buffer_load_") and re.search(r"\blds\b", ops))


def _functions(text):
    """{symbol: listing text} of an llvm-objdump listing (instructions under their '<symbol>:' label)"""
    out, name = {}, None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-fA-F]+ <(.+)>:$", line.strip())
        if m:
            name = m.group(1)
            out[name] = []
        elif name is not None:
            out[name].append(line)
    return {k: "\n".join(v) for k, v in out.items()}


CALLS = re.compile(r"^(s_swappc|s_setpc|s_call)")


def check_listing(text):
    """(M0 writes, LDS DMAs) of one function's listing; AssertionError on any violation of rules 1-3
    when it issues an LDS DMA (functions without one are not constrained)"""
    ins = _instructions(text)
    if not any(_is_lds_dma(mn, ops) for mn, ops in ins):
        return 0, 0
    writes = dmas = 0
    for i, (mn, ops) in enumerate(ins):
        assert not CALLS.match(mn), f"a function with LDS DMA calls another: {mn} {ops}"
        if re.search(r"\bm0\b", ops):
            assert mn == "s_mov_b32" and ops.startswith("m0,"), f"M0 used by {mn} {ops}"
            assert i + 1 < len(ins) and _is_lds_dma(*ins[i + 1]), f"M0 write not followed by an LDS DMA: {ins[i + 1:i + 2]}"
            writes += 1
        if _is_lds_dma(mn, ops):
            prev = ins[i - 1] if i else ("", "")
            assert prev[0] == "s_mov_b32" and prev[1].startswith("m0,"), f"LDS DMA without its M0 write: {mn} {ops}"
            dmas += 1
        assert not IMPLICIT_M0.match(mn), f"instruction reading M0 implicitly: {mn} {ops}"
    return writes, dmas


def test_m0_written_only_right_before_each_lds_dma(disassembly):
    writes = dmas = kernels = 0
    for text in disassembly:
        for name, body in _functions(text).items():
            w, n = check_listing(body)
            writes, dmas, kernels = writes + w, dmas + n, kernels + (n > 0)
    assert writes == dmas and dmas > 0 and kernels >= 4


def test_functions_split_by_symbol():
    text = "0000000000001000 <k1>:\n\ts_nop 0\n\n0000000000002000 <k2>:\n\ts_endpgm\n"
    assert list(_functions(text)) == ["k1", "k2"]


GOOD = """
	s_mov_b32 m0, s4                                 // 000000000100: BEFC0004
	buffer_load_dwordx4 v76, s[12:15], 0 offen lds             // 000000003A40: E05D1000 8003004C
	v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]
	s_mov_b32 m0, s5
	global_load_lds_dwordx4 v[28:29], off
"""


@pytest.mark.parametrize("bad", [
    GOOD.replace("\tv_mfma", "\tv_movrels_b32 v1, v2\n\tv_mfma"),                  # a compiler M0 reader
    GOOD.replace("offen lds", "offen lds\n\ts_sendmsg sendmsg(MSG_DEALLOC_VGPRS)"),    # another one
    GOOD.replace("s_mov_b32 m0, s5\n", "s_mov_b32 m0, s5\n\ts_nop 0\n"),           # a gap
    GOOD.replace("\ts_mov_b32 m0, s4", "\ts_nop 0"),                                  # a DMA without its write
    GOOD + "\tv_readlane_b32 s0, v1, m0\n",                                           # M0 named elsewhere
    GOOD + "\ts_swappc_b64 s[30:31], s[16:17]\n",                                     # a call
    GOOD + "\ts_set_gpr_idx_on s3, gpr_idx(DST)\n",                                  # indexed register access
])
def test_checker_rejects_violations(bad):
    assert check_listing(GOOD) == (2, 2)
    with pytest.raises(AssertionError):
        check_listing(bad)


def test_functions_without_lds_dma_are_free():
    assert check_listing("\ts_set_gpr_idx_on s3, gpr_idx(DST)\n\tv_mov_b32 v1, v2\n") == (0, 0)
