"""The TypeScript host (gemma4-webgpu_amd/host/*.ts) over the N-API addon, run by Node.

CPU: the type-stripping loader turns every host source into JavaScript that
compiles; the kernel table, Params sizes and uniform layout agree with the C
ABI (node host/run.js cpu). The GPU case lives in test_gpu_host_node.py.
"""
import json
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "gemma4-webgpu_amd" / "host"
ADDON = ROOT / "gemma4-webgpu_amd" / "lib" / "g4attn.node"
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_node(*args, timeout=120):
    return subprocess.run([NODE, *args], cwd=ROOT, capture_output=True, text=True, timeout=timeout)


def test_stripped_sources_compile():
    script = (
        "const {strip} = require('./gemma4-webgpu_amd/host/ts_register');"
        "const fs = require('fs'); const vm = require('vm');"
        "for (const f of process.argv.slice(1)) {"
        "  const src = fs.readFileSync(f, 'utf8'); const js = strip(src);"
        "  new vm.Script(js, {filename: f});"
        "  if (js.split('\\n').length < src.split('\\n').length) throw new Error(f + ': lines lost');"
        "  if (/\\binterface\\s+\\w+\\s*\\{/.test(js)) throw new Error(f + ': interface left');"
        "}"
        "console.log('ok');"
    )
    files = sorted(str(p) for p in HOST.glob("*.ts"))
    assert files
    r = run_node("-e", script, *files)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"


def test_stripper_erases_type_syntax():
    src = (
        "import { a } from './x';\\nimport type { T } from './y';\\n"
        "export interface P { x: number; y?: string }\\nexport type U = { u: number } | { f: number };\\n"
        "export function f(x: number, y?: string, z: number = 3): number { const w: number[] = [x]; "
        "return (w[0] as number) + z; }\\n"
        "export class C implements P { private readonly q: number; r: string = 'r';\\n"
        "  constructor(q: number) { this.q = q; }\\n  get(): number { return this.q; } }\\n"
    )
    script = (
        "const {strip} = require('./gemma4-webgpu_amd/host/ts_register');"
        f"const js = strip(\"{src}\");"
        "console.log(JSON.stringify(js));"
    )
    r = run_node("-e", script)
    assert r.returncode == 0, r.stderr
    js = json.loads(r.stdout)
    for gone in ("interface", "type U", ": number", "implements", "private", "readonly", " as ", "y?"):
        assert gone not in js, (gone, js)
    assert "const { a } = require('./x')" in js
    assert "exports.f = f;" in js and "exports.C = C;" in js
    assert re.search(r"\br\s*= 'r';", js)  # field kept with its initialiser, annotation blanked


@pytest.mark.skipif(not ADDON.exists(), reason="g4attn.node not built (no Node headers)")
def test_host_cpu_checks():
    r = run_node(str(HOST / "run.js"), "cpu")
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["ok"] and "uniform layout" in res["checks"]
