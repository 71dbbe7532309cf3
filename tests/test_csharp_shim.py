"""The C# binding under csharp/ (not built in this image, which has no .NET toolchain) checked against the C
ABI it binds: every symbol include/lonnx.h declares has one [DllImport] with the same parameter count, the
blittable structs list the C fields in order, and the HIP twins cover every operator of the reference's
Node.ExecuteCPU switch (src/Lokad.Onnx.Backend/Node.cs:121-181) and CPUExecutionProvider
(CPUExecutionProvider.cs:56-695)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CS = os.path.join(ROOT, "csharp")

# the op cases of Node.ExecuteCPU (Node.cs:121-181), in order
REFERENCE_OPS = ["Reshape", "Add", "Sub", "Mul", "Div", "Pow", "Sqrt", "Conv", "Relu", "Erf", "MaxPool", "MatMul",
                 "Transpose", "Constant", "Cast", "Concat", "Shape", "Gather", "Slice", "Unsqueeze", "ReduceSum",
                 "ReduceMean", "ReduceMax", "Softmax"]


def _header_functions():
    s = open(os.path.join(ROOT, "include", "lonnx.h")).read()
    s = re.sub(r"/\*.*?\*/", "", s, flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:int|int32_t|int64_t|const char \*|void \*)\s*(lx_\w+)\(([^;]*)\);", s, flags=re.M):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _cs(name):
    return open(os.path.join(CS, name)).read()


def test_every_exported_symbol_has_one_dllimport_with_its_arity():
    decl = _header_functions()
    assert len(decl) >= 70
    s = re.sub(r"//[^\n]*", "", _cs("HipNative.cs"))
    found = {}
    for m in re.finditer(r"\[DllImport\(Lib[^\]]*\)\]\s*public static extern [\w\*\[\]\?]+ (lx_\w+)\(([^)]*)\);", s):
        args = " ".join(m.group(2).split())
        found.setdefault(m.group(1), []).append(0 if not args else args.count(",") + 1)
    assert sorted(found) == sorted(decl), (set(decl) ^ set(found))
    for name, n in decl.items():
        assert found[name] == [n], (name, found[name], n)


def test_struct_layouts_follow_the_c_structs():
    s = _cs("HipNative.cs")

    def fields(struct):
        body = re.search(r"struct " + struct + r"\s*\{(.*?)\n\}", s, flags=re.S).group(1)
        return re.findall(r"public (?:fixed )?(\w+) (\w+)(?:\[[^\]]*\])?;", body)
    assert [t for t, _ in fields("LxTensor")] == ["int", "int", "long", "IntPtr", "long", "int", "int"]
    assert [t for t, _ in fields("LxNodeProfile")] == ["long", "int", "byte", "double", "double", "double"]
    assert [t for t, _ in fields("LxOpProfile")] == ["byte", "double", "double", "double"]
    assert "fixed byte Op[36]" in s
    assert [t for t, _ in fields("LxBroadcastPlan")] == ["int", "int", "long", "int", "int", "long", "long", "long", "long"]


def test_execute_hip_switch_covers_every_execute_cpu_case():
    s = _cs("Node.ExecuteHIP.cs")
    cases = re.findall(r"OpType\.(\w+) =>", s)
    assert cases == REFERENCE_OPS
    assert "_ => NotSupported(Op)" in s


def test_provider_has_a_twin_of_every_operator():
    s = _cs("HipExecutionProvider.cs")
    methods = set(re.findall(r"public static OpResult (\w+)\(", s))
    assert set(REFERENCE_OPS) <= methods, set(REFERENCE_OPS) - methods


def test_sources_are_balanced():
    for f in os.listdir(CS):
        s = re.sub(r'"(?:[^"\\]|\\.)*"', '""', re.sub(r"//[^\n]*", "", _cs(f)))
        for o, c in ("{}", "()", "[]"):
            assert s.count(o) == s.count(c), (f, o)


def test_provider_opens_a_device_math_stage_before_every_native_operator_call():
    """With Profiler.Enabled the provider opens OpStage.Math as the reference's operators do
    (CPUExecutionProvider.cs:92-103), right before each native operator call (after the uploads), and later
    writes the device time the library recorded for that call into that OpProfile."""
    s = re.sub(r"//[^\n]*", "", _cs("HipExecutionProvider.cs"))
    body = s[s.index("static void MathStage()"):]
    body = body[:body.index("\n    }\n") + 6]
    assert "if (!Profiler.Enabled) return;" in body
    assert "HipNative.lx_set_op_profiling(1)" in body
    assert "Profiler.StartOpStage(OpStage.Math);" in body
    assert "pendingMath.Add((Profiler.CurrentOpProfile, HipNative.lx_op_profile_count()));" in body
    resolve = s[s.index("public static void ResolveDeviceProfile()"):]
    resolve = resolve[:resolve.index("\n    }\n")]
    assert "HipNative.lx_op_profile(record, &p)" in resolve and "stage.Time = TimeSpan.FromMilliseconds(p.MathMs);" in resolve
    assert "HipNative.lx_op_profile_reset()" in resolve
    lines = s.split("\n")
    calls = [i for i, l in enumerate(lines)
             if re.search(r"(st = |Done\(op, )(HipNative\.lx_[A-Z]\w*|fn)\(&", l) or "HipNative.lx_Concat(" in l]
    assert len(calls) == 15
    for i in calls:
        back = "\n".join(lines[max(0, i - 6):i + 1])
        assert "MathStage();" in back, lines[i]


def test_every_fused_op_is_charted_under_a_reference_op():
    """HipGraph.FusedOp charts each fused node the graph runtime can make (lx_graph.cpp) under an OpType;
    ElementwiseChain takes the default arm."""
    src = open(os.path.join(ROOT, "onnx_amd", "csrc", "lx_graph.cpp")).read()
    made = set(re.findall(r'(?:f\.|f->)op = "(\w+)"', src))
    assert {"GeluErf", "LayerNormDecomposed", "MatMulAdd", "MatMulAddGroup", "MatMulPermuted", "Attention"} <= made
    s = _cs("HipGraph.cs")
    body = s[s.index("static OpType FusedOp(string name)"):]
    body = body[:body.index("};")]
    charted = set(re.findall(r'"(\w+)"', body))
    assert made - {"ElementwiseChain"} <= charted, made - charted
