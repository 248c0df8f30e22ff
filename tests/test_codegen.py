"""Wait counts of the stream, split-K and decode GEMV kernels, checked in the
built gfx950 code (llvm-objdump of the plugin's own code objects).

Each of these kernels copies x (and scales) into LDS by buffer->LDS DMA,
then issues its weight loads into registers, then waits with
`s_waitcnt vmcnt(n)` for n = the number of those weight loads and crosses
a barrier: the wait means "every DMA before them has landed" only if all n
register loads are issued before it.  The compiler may still move a load
into a later, lane-conditional block (it did once, for a per-lane select of
the partial sums), and then the wait silently stops covering the DMA.  This
test counts, per kernel, the register-returning buffer loads issued before
the first `s_barrier` and checks them against the wait's count.

The other checks here read the same code objects: issue order of the
whole-line kernels, the split-K GEMM's in-flight loads, and that no kernel
of the plugin spills registers to scratch memory.
"""
import os
import re
import shutil
import subprocess

import pytest

LLVM = "/opt/rocm/llvm/bin"
KERNELS = ("qgemv_stream_kernel", "qgemv_split_kernel", "qgemv_dec_kernel", "qmm_skinny_kernel")
LINE = "qgemv_line_kernel"
MX = "qgemv_mx_kernel"
Q4 = "qgemv_q4_kernel"
SK = "qgemm_sk_kernel"


def _tool(name):
    p = os.path.join(LLVM, name)
    return p if os.path.exists(p) else shutil.which(name)


@pytest.fixture(scope="module")
def code_objects(tmp_path_factory):
    """The plugin's embedded gfx950 code objects, unpacked into a temp dir.

    The plugin stores them as compressed offload bundles ("CCOB" header:
    magic, u16 version, u16 method, then the bundle's total size, u64 in
    version 3, u32 before) in its .hip_fatbin section; each bundle is cut
    out at its stated size and unbundled by clang-offload-bundler."""
    import struct

    import mlx_amd
    objdump, objcopy, bundler = _tool("llvm-objdump"), _tool("llvm-objcopy"), _tool("clang-offload-bundler")
    if not (objdump and objcopy and bundler):
        pytest.skip("llvm-objdump / llvm-objcopy / clang-offload-bundler not available")
    assert os.path.exists(mlx_amd.PLUGIN_PATH), "run __graft_entry__.build() first"
    d = tmp_path_factory.mktemp("codeobj")
    fat = d / "fatbin.bin"
    subprocess.run([objcopy, "-O", "binary", "--only-section=.hip_fatbin", mlx_amd.PLUGIN_PATH, str(fat)],
                   check=True, capture_output=True)
    data = fat.read_bytes()
    cos, i = [], data.find(b"CCOB")
    while i >= 0:
        ver = struct.unpack_from("<H", data, i + 4)[0]
        size = struct.unpack_from("<Q" if ver >= 3 else "<I", data, i + 8)[0]
        src, out = d / f"b{len(cos)}.ccob", d / f"b{len(cos)}.gfx950.co"
        src.write_bytes(data[i:i + size])
        subprocess.run([bundler, "--unbundle", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--input={src}", f"--output={out}"], check=True, capture_output=True)
        cos.append(out)
        i = data.find(b"CCOB", i + size)
    if not cos:  # uncompressed bundles: --offloading writes them next to its input
        so = d / "plugin.so"
        shutil.copy(mlx_amd.PLUGIN_PATH, so)
        subprocess.run([objdump, "--offloading", str(so)], cwd=d, check=True, capture_output=True)
        cos = sorted(d.glob("plugin.so.*gfx950*"))
    assert cos, "no gfx950 code object in the plugin"
    return cos


@pytest.fixture(scope="module")
def disassembly(code_objects):
    objdump = _tool("llvm-objdump")
    out = {}
    for co in code_objects:
        syms = subprocess.run([objdump, "-t", str(co)], check=True, capture_output=True, text=True).stdout
        names = [ln.split()[-1] for ln in syms.splitlines()
                 if " .text" in ln and any(k in ln for k in KERNELS + (LINE, MX, Q4, SK)) and not ln.endswith(".kd")]
        if not names:
            continue
        dis = subprocess.run([objdump, "-d", "--mcpu=gfx950", "--disassemble-symbols=" + ",".join(names), str(co)],
                             check=True, capture_output=True, text=True).stdout
        cur = None
        for ln in dis.splitlines():
            m = re.match(r"^[0-9a-f]+ <(\S+)>:", ln)
            if m:
                cur = m.group(1)
                out[cur] = []
            elif cur and ln.strip():
                out[cur].append(ln.strip())
    return out


def test_weight_loads_precede_their_wait(disassembly):
    found = {k: 0 for k in KERNELS}
    bad = []
    for name, lines in disassembly.items():
        if LINE in name or MX in name or Q4 in name or SK in name:
            continue
        loads, vm = 0, None
        for t in lines:
            if t.startswith("buffer_load") and not re.search(r"\blds\b", t):
                loads += 1
            m = re.search(r"s_waitcnt\b.*\bvmcnt\((\d+)\)", t)
            if m:
                vm = int(m.group(1))
            if t.startswith("s_barrier"):
                break
        else:
            continue  # no barrier: nothing to check
        for k in KERNELS:
            found[k] += k in name
        if vm is not None and loads < vm:
            bad.append(f"{name}: {loads} loads before vmcnt({vm})")
    assert all(found.values()), f"kernels not found in the plugin: {found}"
    assert not bad, "\n".join(bad[:10])


def test_line_kernel_issue_order(disassembly):
    """The whole-line kernels (M = 1, and the K-split one for 2..4 rows of x)
    and the 4x4x4-MFMA decode kernel, which loads in the same order:
    x and scale loads (default cache policy) all issue before the block
    barrier, the non-temporal code loads all after it and before the first
    wait on a vector-memory load -- so the x and scale requests of every wave
    precede the codes in the CU's queue, and no code load was moved behind
    the arithmetic.  One exception: the M = 1 kernel with 7 rows per wave and
    its own x (4-bit codes, 16-bit x) issues its first row's NI code loads
    first, ahead of every x and scale load."""
    seen, seen_mx, seen_q4, seen_early, bad = 0, 0, 0, 0, []
    for name, lines in disassembly.items():
        if LINE not in name and MX not in name and Q4 not in name:
            continue
        seen += 1
        seen_mx += MX in name
        seen_q4 += Q4 in name
        bar = next((i for i, t in enumerate(lines) if t.startswith("s_barrier")), None)
        if bar is None:
            bad.append(f"{name}: no barrier")
            continue
        before, after = lines[:bar], lines[bar:]
        # template arguments <BITS, TX, SB, R, NI, ...> of the whole-line kernel
        m = re.search(LINE + r"ILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)E", name)
        early = 0
        if m:
            bits, tx, r, ni = int(m.group(1)), int(m.group(2)), int(m.group(4)), int(m.group(5))
            if bits == 4 and tx != 0 and r == 7:
                early = ni
                seen_early += 1
        loads = [t for t in before if t.startswith("buffer_load")]
        nt = [re.search(r"\bnt\b", t) is not None for t in loads]
        if nt != [True] * early + [False] * (len(loads) - early):
            bad.append(f"{name}: {sum(nt)} code loads before the barrier (expected the first {early})")
        if not any(t.startswith("buffer_load") for t in before):
            bad.append(f"{name}: no x/scale load before the barrier")
        wait = next((i for i, t in enumerate(after) if re.search(r"s_waitcnt\b.*\bvmcnt\(", t)), len(after))
        late = [t for t in after[wait:] if t.startswith("buffer_load")]
        if late:
            bad.append(f"{name}: {len(late)} loads after the first vmcnt wait")
        if not any(t.startswith("buffer_load") and re.search(r"\bnt\b", t) for t in after[:wait]):
            bad.append(f"{name}: no code load between the barrier and the first wait")
    assert seen and seen_mx and seen_q4, "qgemv_line_kernel, qgemv_mx_kernel or qgemv_q4_kernel not found in the plugin"
    assert seen_early, "no 7-row whole-line kernel with its own x found in the plugin"
    assert not bad, "\n".join(bad[:10])


def test_split_k_gemm_keeps_loads_in_flight(disassembly):
    """The split-K small-M GEMM: (1) no L2 writeback or invalidate anywhere
    (its partial sums cross XCDs through device-scope cache-policy loads and
    stores; a device-scope fence there made launches 4-5x slower); (2) in the
    main loop (the super-steps between the prologue's barrier and the fourth
    after it) every wait leaves at least 8 vector-memory loads in flight: a
    load the compiler cannot count (one issued on only some paths) makes it
    drain them all before every super-step."""
    seen, bad = 0, []
    for name, lines in disassembly.items():
        if SK not in name:
            continue
        seen += 1
        if any(t.startswith(("buffer_wbl2", "buffer_inv")) for t in lines):
            bad.append(f"{name}: L2 writeback/invalidate")
        bars = [i for i, t in enumerate(lines) if t.startswith("s_barrier")]
        if len(bars) < 5:
            bad.append(f"{name}: {len(bars)} barriers")
            continue
        low = [int(m.group(1)) for t in lines[bars[0]:bars[4]]
               for m in [re.search(r"s_waitcnt\b.*\bvmcnt\((\d+)\)", t)] if m and int(m.group(1)) < 8]
        if low:
            bad.append(f"{name}: main-loop waits down to vmcnt({min(low)})")
    assert seen, "qgemm_sk_kernel not found in the plugin"
    assert not bad, "\n".join(bad[:10])


def test_no_kernel_spills_to_scratch(code_objects):
    """Every kernel of the plugin runs without a private (scratch) segment:
    a register spill there turns into per-lane memory traffic and a full
    vector-memory drain (a spilled load's value has to arrive before it can
    be stored), and on these streaming kernels that costs more than the
    spill saves.  Spills into the accumulator registers (no memory) are
    allowed."""
    readelf = _tool("llvm-readelf")
    if not readelf:
        pytest.skip("llvm-readelf not available")
    seen, bad = 0, []
    for co in code_objects:
        notes = subprocess.run([readelf, "--notes", str(co)], check=True, capture_output=True, text=True).stdout
        # one YAML map per kernel in .amdhsa.kernels; each holds .name and
        # .private_segment_fixed_size
        # (kernel entries at indent 2, their keys at 4, argument entries deeper)
        for block in re.split(r"\n  - \.", notes):
            name = re.search(r"^    \.name:\s+(\S+)", block, re.M)
            priv = re.search(r"^    \.private_segment_fixed_size:\s+(\d+)", block, re.M)
            if not name or not priv:
                continue
            seen += 1
            if int(priv.group(1)):
                bad.append(f"{name.group(1)}: {priv.group(1)} bytes of scratch per lane")
    assert seen > 100, f"only {seen} kernels found in the code objects' metadata"
    assert not bad, f"{len(bad)} kernels spill:\n" + "\n".join(bad[:10])
