// Checks of the TypeScript host over the N-API addon, driven by tests/test_host_node.py.
//
//   node host/run.js cpu            layout and table checks (no GPU work)
//   node host/run.js layer <dir>    one attention layer from <dir>/case.json + case.bin, run twice on the
//                                   GPU: the engine's six dispatches in order (src/engine.ts:2056-2094),
//                                   and the fused attnStep; results go to <dir>/out.bin for the oracle check.
//   node host/run.js promptprep <dir>  the chunked prompt prep of one producer layer from <dir>/case.json +
//                                   case.bin; q_out and both caches go to <dir>/out.bin.
//   node host/run.js prefill <dir>  two prefill chunks (entries) from <dir>/case.json + case.bin in one
//                                   attnPrefill call; outputs go to <dir>/out.bin.
//   node host/run.js head <dir>     the sampling head from <dir>/case.json + case.bin: the engine's lmHead,
//                                   logitSoftcap and sample.argmax dispatches (src/engine.ts:2223-2255),
//                                   then the fused lmHeadArgmax; results go to <dir>/out.bin.
//   node host/run.js batch <dir>    continuous batching from <dir>/case.json + case.bin: sequences are
//                                   submitted, admitted into cache slots and released over several token
//                                   steps of a DecodeScheduler, one attnStep per layer over the active
//                                   sequences; every attnOut goes to <dir>/out.bin, in step, layer and
//                                   admission order.
//   node host/run.js readback <dir> f32 values from <dir>/case.bin: logitSoftcap in place, then two
//                                   readBufferAsync calls around a clearBuffer; both results (the
//                                   softcapped values, then zeros) go to <dir>/out.bin.
//   node host/run.js capture <dir>  captureAttention at each per-layer capture point of a producer and a
//                                   consumer layer from <dir>/case.json + case.bin; results to <dir>/out.bin.
//   node host/run.js linear <dir>   the projections from <dir>/case.json + case.bin: one matmulQuant
//                                   dispatch per weight matrix (attn.linearQKV, src/engine.ts:2045-2051),
//                                   then one linear call over all of them; results go to <dir>/out.bin.

import { BINDINGS, KERNELS, PARAMS_BYTES, PASS_LABELS, Uniform, HipAttention, loadAddon } from './attention';
import type { DeviceBuffer, KernelName } from './attention';
import { DecodeScheduler, SlotTable } from './scheduler';

declare const require: any;
declare const process: any;

const fs = require('fs');
const path = require('path');

function fail(msg: string): never {
  throw new Error(msg);
}

function throws(f: () => void, what: string): void {
  let threw = false;
  try {
    f();
  } catch (e) {
    threw = true;
  }
  if (!threw) fail(`expected an error: ${what}`);
}

function same(a: any, b: any, what: string): void {
  if (JSON.stringify(a) !== JSON.stringify(b)) fail(`${what}: ${JSON.stringify(a)} != ${JSON.stringify(b)}`);
}

// The continuous-batching bookkeeping: FIFO admission into the lowest free slot, release and reuse,
// the per-token advance, and the errors.
function slotTableChecks(): void {
  const t = new SlotTable(2, 10);
  t.submit('a', 3);
  t.submit('b', 0);
  t.submit('c', 9);
  same(t.admit(), ['a', 'b'], 'first admission');
  same(t.activeIds(), ['a', 'b'], 'active');
  same(t.waitingIds(), ['c'], 'waiting');
  same([t.slotOf('a'), t.slotOf('b')], [0, 1], 'slots');
  same(t.admit(), [], 'no free slot');
  t.release('a');
  same(t.admit(), ['c'], 'admission after release');
  same(t.slotOf('c'), 0, 'freed slot reused');
  same(t.activeIds(), ['b', 'c'], 'admission order');
  throws(function () { t.submit('b', 1); }, 'duplicate id');
  throws(function () { t.submit('d', 10); }, 'length beyond the cache');
  throws(function () { t.submit('d', -1); }, 'negative length');
  t.advance();
  same([t.lengthOf('b'), t.lengthOf('c')], [1, 10], 'advance');
  if (!t.isFull('c') || t.isFull('b')) fail('isFull');
  throws(function () { t.advance(); }, 'advance past a full sequence');
  same([t.lengthOf('b'), t.lengthOf('c')], [1, 10], 'a failed advance changes nothing');
  throws(function () { t.release('zz'); }, 'unknown id');
  t.submit('d', 2);
  t.submit('e', 2);
  t.release('d');
  same(t.waitingIds(), ['e'], 'release of a waiting request');
  t.release('b');
  t.release('c');
  same(t.admit(), ['e'], 'admission into an empty table');
  same(t.slotOf('e'), 0, 'lowest free slot first');
  throws(function () { t.lengthOf('b'); }, 'released sequence');
  throws(function () { return new SlotTable(0, 4); }, 'zero capacity');
}

export function cpuChecks(): string[] {
  const done: string[] = [];
  const g4 = loadAddon();
  const names = Object.keys(BINDINGS).sort();
  if (Object.keys(KERNELS).sort().join() !== names.join()) fail('KERNELS and BINDINGS name different kernels');
  for (const n of names) if (!PASS_LABELS[n]) fail(`no pass label for ${n}`);
  done.push('kernel table');
  const sizes: Record<string, string> = {
    fusedPerHeadNormRope: 'sizeofNormRopeParams', perHeadRmsNormNoWeight: 'sizeofNormParams',
    kvCacheStore: 'sizeofKvStoreParams', attnScore: 'sizeofAttnScoreParams', softmax: 'sizeofSoftmaxParams',
    attnOutput: 'sizeofAttnOutputParams', matmulQuant: 'sizeofMatmulParams', logitSoftcap: 'sizeofSoftcapParams',
    matmulQ8: 'sizeofMatmulParams', matmulQ4K: 'sizeofMatmulParams',
    argmax: 'sizeofArgmaxParams',
  };
  for (const n of names) {
    const want = g4[sizes[n]];
    const have = PARAMS_BYTES[n as KernelName];
    if (have !== want) fail(`${n}: params ${have} B, C struct ${want} B`);
  }
  done.push('params sizes');
  // Uniform layout: the engine's fusedNormRopeQ list, then the per-token position patch at byte 12.
  const u = new Uniform([{ u: 8 }, { u: 256 }, { f: 1e-6 }, { u: 0 }, { f: 1e4 }, { u: 1 }]);
  u.writeU32(12, 8192);
  const dv = new DataView(u.bytes.buffer);
  if (dv.getUint32(0, true) !== 8 || dv.getUint32(4, true) !== 256 || dv.getUint32(12, true) !== 8192 ||
    dv.getUint32(20, true) !== 1 || Math.abs(dv.getFloat32(8, true) - 1e-6) > 1e-12 || dv.getFloat32(16, true) !== 1e4) {
    fail('uniform layout');
  }
  if (new Uniform([{ u: 1 }]).bytes.byteLength !== 16) fail('uniforms are padded to 16 bytes');
  done.push('uniform layout');
  slotTableChecks();
  done.push('slot table');
  if (typeof g4.version() !== 'string') fail('version');
  done.push('addon loaded: ' + g4.version());
  // attnStepRunPair takes two 64-byte plans; anything else is refused before the library is called
  throws(() => g4.attnStepRunPair(new Uint8Array(3), new Uint8Array(64), BigInt(0)), 'attnStepRunPair: short plan');
  done.push('step pair arguments');
  if (g4.sizeofPromptPrepEntry() !== 128) fail(`g4_prompt_prep_entry is ${g4.sizeofPromptPrepEntry()} B, the host writes 128`);
  throws(() => g4.attnPromptPrepMany(new Uint8Array(100), 1, BigInt(0)), 'attnPromptPrepMany: short record');
  done.push('prompt prep records');
  return done;
}

interface CaseSpec {
  nqh: number; nkh: number; hd: number; seq: number; pos: number; window: number; theta: number; div: number;
  eps: number; oRows: number; arrays: Record<string, number[]>;
}

function layer(dir: string): string[] {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as CaseSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const NQH = spec.nqh, NKH = spec.nkh, HD = spec.hd, SEQ = spec.seq;
  const bufs: DeviceBuffer[] = [];
  function upload(name: string): DeviceBuffer {
    const r = spec.arrays[name];
    const b = att.createBuffer(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    bufs.push(b);
    return b;
  }
  function alloc(bytes: number): DeviceBuffer {
    const b = att.createBuffer(bytes);
    bufs.push(b);
    return b;
  }
  const qw = upload('qw'), kw = upload('kw'), rf = upload('rf');

  // (1) the engine's order over the six kernels, uniforms built as the engine builds them
  const q1 = upload('q'), k1 = upload('k'), v1 = upload('v'), kc1 = upload('kc'), vc1 = upload('vc');
  const scores = alloc(NQH * SEQ * 4), out1 = alloc(NQH * HD * 4);
  const vNorm = new Uniform([{ u: NKH }, { u: HD }, { f: spec.eps }, { u: 0 }]);
  const normRopeQ = new Uniform([{ u: NQH }, { u: HD }, { f: spec.eps }, { u: 0 }, { f: spec.theta }, { u: spec.div }]);
  const normRopeK = new Uniform([{ u: NKH }, { u: HD }, { f: spec.eps }, { u: 0 }, { f: spec.theta }, { u: spec.div }]);
  const kvStore = new Uniform([{ u: NKH }, { u: HD }, { u: 0 }, { u: SEQ }]);
  const score = new Uniform([{ u: NQH }, { u: NKH }, { u: HD }, { u: 0 }, { f: 1.0 }, { u: spec.window }]);
  const softmax = new Uniform([{ u: NQH }, { u: 0 }]);
  const output = new Uniform([{ u: NQH }, { u: NKH }, { u: HD }, { u: 0 }]);
  // per-token patches (src/engine.ts:1977-1987)
  normRopeQ.writeU32(12, spec.pos);
  normRopeK.writeU32(12, spec.pos);
  kvStore.writeU32(8, spec.pos);
  score.writeU32(12, SEQ);
  softmax.writeU32(4, SEQ);
  output.writeU32(12, SEQ);
  att.dispatch('perHeadRmsNormNoWeight', [v1], vNorm);
  att.dispatch('fusedPerHeadNormRope', [q1, qw, rf], normRopeQ);
  att.dispatch('fusedPerHeadNormRope', [k1, kw, rf], normRopeK);
  att.dispatch('kvCacheStore', [k1, v1, kc1, vc1], kvStore);
  att.dispatch('attnScore', [q1, kc1, scores], score);
  att.dispatch('softmax', [scores], softmax);
  att.dispatch('attnOutput', [scores, vc1, out1], output);

  // (2) the fused step on fresh copies of the same inputs, with the RoPE table
  const q2 = upload('q'), k2 = upload('k'), v2 = upload('v'), kc2 = upload('kc'), vc2 = upload('vc');
  const out2 = alloc(NQH * HD * 4);
  const rfr = spec.arrays['rf'];
  const rfBits = new Uint16Array(rfr[1] / 2);
  new Uint8Array(rfBits.buffer).set(bin.subarray(rfr[0], rfr[0] + rfr[1]));
  const inv = att.ropeInvFreqHost(spec.theta, HD, spec.div, rfBits);
  const shape = { numQHeads: NQH, numKvHeads: NKH, headDim: HD };
  const ws = alloc(att.attnStepWorkspaceSize(1, shape));
  att.attnStep([{
    q: q2, k: k2, v: v2, qWeight: qw, kWeight: kw, ropeFreqs: rf, ropeInvFreq: inv, kCache: kc2, vCache: vc2,
    out: out2, seqLen: SEQ, position: spec.pos, slidingWindow: spec.window, storeKv: true, theta: spec.theta,
    applyDivisor: spec.div, scale: 1.0, eps: spec.eps,
  }], shape, ws);

  // (3) the same step as attention pass + attn.linearOut with the merge folded in, and linear() over (2)'s attnOut
  const q3 = upload('q'), k3 = upload('k'), v3 = upload('v'), kc3 = upload('kc'), vc3 = upload('vc');
  const out3 = alloc(NQH * HD * 4), wo = upload('wo');
  const R = spec.oRows;
  const y3 = alloc(R * 4), y2 = alloc(R * 4);
  const ws3 = alloc(att.attnStepWorkspaceSize(1, shape));
  const plan3 = att.attnStepPrepare([{
    q: q3, k: k3, v: v3, qWeight: qw, kWeight: kw, ropeFreqs: rf, ropeInvFreq: inv, kCache: kc3, vCache: vc3,
    out: out3, seqLen: SEQ, position: spec.pos, slidingWindow: spec.window, storeKv: true, theta: spec.theta,
    applyDivisor: spec.div, scale: 1.0, eps: spec.eps,
  }], shape, ws3);
  att.attnStepRunAttention(plan3);
  att.attnStepOut(plan3, shape, [{ weight: wo, out: y3, rows: R }]);
  att.linear(out2, NQH * HD, [{ weight: wo, out: y2, rows: R }]);

  // (4) two layers of one token prepared together (one upload, one RoPE set for both), each on fresh copies of
  // the inputs: the first run as attention + merge, the second as attention + attn.linearOut
  const step4 = [0, 1].map(function () {
    return {
      q: upload('q'), k: upload('k'), v: upload('v'), qWeight: qw, kWeight: kw, ropeFreqs: rf, ropeInvFreq: inv,
      kCache: upload('kc'), vCache: upload('vc'), out: alloc(NQH * HD * 4), seqLen: SEQ, position: spec.pos,
      slidingWindow: spec.window, storeKv: true, theta: spec.theta, applyDivisor: spec.div, scale: 1.0,
      eps: spec.eps,
    };
  });
  const y4 = alloc(R * 4);
  const plans4 = att.attnStepPrepareLayers(step4, shape, alloc(att.attnStepLayersWorkspaceSize(2, shape)));
  att.attnStepRun(plans4[0]);
  att.attnStepRunAttention(plans4[1]);
  att.attnStepOut(plans4[1], shape, [{ weight: wo, out: y4, rows: R }]);

  // results: out1, out2, out3 (f32), y2, y3 (f32), the stored row of kc1, vc1, kc2, vc2 (f16), then (4)'s two
  // attnOut (f32), its y (f32) and its layers' stored rows (k, v of each, f16)
  const row = NKH * HD * 2, o = NQH * HD * 4, yb = R * 4;
  const res = new Uint8Array(3 * o + 2 * yb + 4 * row + 2 * o + yb + 4 * row);
  att.readBuffer(out1, 0, res.subarray(0, o));
  att.readBuffer(out2, 0, res.subarray(o, 2 * o));
  att.readBuffer(out3, 0, res.subarray(2 * o, 3 * o));
  att.readBuffer(y2, 0, res.subarray(3 * o, 3 * o + yb));
  att.readBuffer(y3, 0, res.subarray(3 * o + yb, 3 * o + 2 * yb));
  const base = 3 * o + 2 * yb;
  const caches = [kc1, vc1, kc2, vc2];
  for (let i = 0; i < 4; i++) att.readBuffer(caches[i], spec.pos * row, res.subarray(base + i * row, base + (i + 1) * row));
  const b4 = base + 4 * row;
  att.readBuffer(step4[0].out, 0, res.subarray(b4, b4 + o));
  att.readBuffer(step4[1].out, 0, res.subarray(b4 + o, b4 + 2 * o));
  att.readBuffer(y4, 0, res.subarray(b4 + 2 * o, b4 + 2 * o + yb));
  const c4 = [step4[0].kCache, step4[0].vCache, step4[1].kCache, step4[1].vCache];
  for (let i = 0; i < 4; i++) {
    const at = b4 + 2 * o + yb + i * row;
    att.readBuffer(c4[i], spec.pos * row, res.subarray(at, at + row));
  }
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return ['engine order: 7 dispatches', 'attnStep: 1 entry', 'attnStepOut: 1 entry', 'attnStepPrepareLayers: 2 layers',
    'results written'];
}

interface PrefillSpec {
  nqh: number; nkh: number; hd: number;
  chunks: { start: number; nTokens: number; window: number; q: number[]; kc: number[]; vc: number[] }[];
}

function prefill(dir: string): string[] {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as PrefillSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const bufs: DeviceBuffer[] = [];
  function upload(r: number[]): DeviceBuffer {
    const b = att.createBuffer(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    bufs.push(b);
    return b;
  }
  const outs: DeviceBuffer[] = [];
  const entries = spec.chunks.map(function (c) {
    const out = att.createBuffer(c.nTokens * spec.nqh * spec.hd * 4);
    bufs.push(out);
    outs.push(out);
    return {
      q: upload(c.q), kCache: upload(c.kc), vCache: upload(c.vc), out: out, nTokens: c.nTokens, start: c.start,
      slidingWindow: c.window, scale: 1.0,
    };
  });
  const shape = { numQHeads: spec.nqh, numKvHeads: spec.nkh, headDim: spec.hd };
  const ws = att.createBuffer(Math.max(att.attnPrefillWorkspaceSize(entries, shape), 1));
  bufs.push(ws);
  att.attnPrefill(entries, shape, ws);
  let total = 0;
  for (const o of outs) total += o.size;
  const res = new Uint8Array(total);
  let off = 0;
  for (const o of outs) {
    att.readBuffer(o, 0, res.subarray(off, off + o.size));
    off += o.size;
  }
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return ['attnPrefill: ' + entries.length + ' entries', 'results written'];
}

interface PromptPrepSpec {
  nqh: number; nkh: number; hd: number; start: number; nTokens: number; theta: number; div: number; rows: number;
  vt?: boolean; arrays: Record<string, number[]>;
}

// The chunked prompt prep of one producer layer; out.bin = q_out, then the whole K and V caches.
function promptPrep(dir: string): string[] {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as PromptPrepSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const bufs: DeviceBuffer[] = [];
  function upload(r: number[]): DeviceBuffer {
    const b = att.createBuffer(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    bufs.push(b);
    return b;
  }
  function alloc(bytes: number): DeviceBuffer {
    const b = att.createBuffer(bytes);
    att.clearBuffer(b);
    bufs.push(b);
    return b;
  }
  const A = spec.arrays;
  const qOut = alloc(spec.nTokens * spec.nqh * spec.hd * 2);
  const kc = alloc(spec.rows * spec.nkh * spec.hd * 2);
  const vc = alloc(spec.rows * spec.nkh * spec.hd * 2);
  const rf = upload(A.rf);
  const inv = alloc(spec.hd / 2 * 4);  // the layer's inverse frequencies, computed once (as at load)
  att.ropeInvFreq(spec.theta, spec.hd, spec.div, rf, inv);
  const shape = { numQHeads: spec.nqh, numKvHeads: spec.nkh, headDim: spec.hd };
  // with spec.vt: the V rows also as V^T blocks, then the chunk's prefill reading V from them
  const vt = spec.vt ? alloc(Math.ceil(spec.rows / 32) * 32 * spec.nkh * spec.hd * 2) : undefined;
  att.attnPromptPrep({
    q: upload(A.q), k: upload(A.k), v: upload(A.v), qWeight: upload(A.qw), kWeight: upload(A.kw),
    ropeFreqs: rf, ropeInvFreq: inv, qOut: qOut, kCache: kc, vCache: vc, nTokens: spec.nTokens, start: spec.start,
    theta: spec.theta, applyDivisor: spec.div, maxSeqLen: spec.rows, vtCache: vt,
  }, shape);
  // the same chunk through attnPromptPrepMany (one entry) into fresh buffers: the same bits
  const qOut2 = alloc(qOut.size), kc2 = alloc(kc.size), vc2 = alloc(vc.size);
  const vt2 = vt ? alloc(vt.size) : undefined;
  att.attnPromptPrepMany([{
    q: upload(A.q), k: upload(A.k), v: upload(A.v), qWeight: upload(A.qw), kWeight: upload(A.kw),
    ropeFreqs: rf, ropeInvFreq: inv, qOut: qOut2, kCache: kc2, vCache: vc2, nTokens: spec.nTokens, start: spec.start,
    theta: spec.theta, applyDivisor: spec.div, maxSeqLen: spec.rows, vtCache: vt2,
  }], shape);
  const pairs: DeviceBuffer[][] = [[qOut, qOut2], [kc, kc2], [vc, vc2]];
  if (vt && vt2) pairs.push([vt, vt2]);
  for (const [x, y] of pairs) {
    const bx = new Uint8Array(x.size), by = new Uint8Array(y.size);
    att.readBuffer(x, 0, bx);
    att.readBuffer(y, 0, by);
    for (let i = 0; i < bx.length; i++) if (bx[i] !== by[i]) fail(`attnPromptPrepMany differs at byte ${i}`);
  }
  const parts: DeviceBuffer[] = [qOut, kc, vc];
  if (vt) {
    const out = alloc(spec.nTokens * spec.nqh * spec.hd * 4);
    const entries = [{ q: qOut, kCache: kc, vCache: vc, out: out, nTokens: spec.nTokens, start: spec.start,
      vtCache: vt, vtRows: spec.rows }];
    const ws = alloc(Math.max(att.attnPrefillWorkspaceSize(entries, shape), 1));
    att.attnPrefill(entries, shape, ws);
    parts.push(vt, out);
  }
  let total = 0;
  for (const b of parts) total += b.size;
  const res = new Uint8Array(total);
  let off = 0;
  for (const b of parts) {
    att.readBuffer(b, 0, res.subarray(off, off + b.size));
    off += b.size;
  }
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return ['attnPromptPrep: ' + spec.nTokens + ' tokens' + (vt ? ', V^T blocks, attnPrefill through them' : ''),
    'attnPromptPrepMany: same bits', 'results written'];
}

interface HeadSpec {
  vocab: number; hidden: number; cap: number; arrays: Record<string, number[]>;
}

function head(dir: string): string[] {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as HeadSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const V = spec.vocab, H = spec.hidden;
  const bufs: DeviceBuffer[] = [];
  function upload(name: string): DeviceBuffer {
    const r = spec.arrays[name];
    const b = att.createBuffer(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    bufs.push(b);
    return b;
  }
  function alloc(bytes: number): DeviceBuffer {
    const b = att.createBuffer(bytes);
    bufs.push(b);
    return b;
  }
  const x = upload('x'), w = upload('w');
  // (1) the engine's three passes, uniforms as createUniformBuffers builds them
  const logits1 = alloc(V * 4), res1 = alloc(16);
  att.dispatch('matmulQuant', [x, w, logits1], new Uniform([{ u: V }, { u: H }]));
  if (spec.cap > 0) att.dispatch('logitSoftcap', [logits1], new Uniform([{ u: V }, { f: spec.cap }]));
  att.dispatch('argmax', [logits1, res1], new Uniform([{ u: V }]));
  // (2) the fused pass
  const logits2 = alloc(V * 4), res2 = alloc(16);
  const shape = { vocab: V, hidden: H, cap: spec.cap };
  const ws = alloc(att.lmHeadWorkspaceSize(shape));
  att.lmHeadArgmax(x, w, logits2, res2, ws, shape);
  // results: logits1, logits2 (f32), then result1, result2 (u32)
  const res = new Uint8Array(2 * V * 4 + 8);
  att.readBuffer(logits1, 0, res.subarray(0, V * 4));
  att.readBuffer(logits2, 0, res.subarray(V * 4, 2 * V * 4));
  att.readBuffer(res1, 0, res.subarray(2 * V * 4, 2 * V * 4 + 4));
  att.readBuffer(res2, 0, res.subarray(2 * V * 4 + 4, 2 * V * 4 + 8));
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return ['engine order: 3 dispatches', 'lmHeadArgmax: 1 call', 'results written'];
}

interface LinearSpec {
  n: number; rows: number[]; format?: string; arrays: Record<string, number[]>;
}

function linear(dir: string): string[] {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as LinearSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const bufs: DeviceBuffer[] = [];
  function alloc(bytes: number): DeviceBuffer {
    const b = att.createBuffer(bytes);
    bufs.push(b);
    return b;
  }
  function upload(name: string): DeviceBuffer {
    const r = spec.arrays[name];
    const b = alloc(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    return b;
  }
  const x = upload('x');
  const fmt = spec.format || 'f16';
  const ws = spec.rows.map(function (_r, i) { return upload('w' + i); });
  const metas = fmt === 'f16' ? [] : spec.rows.map(function (_r, i) { return upload('m' + i); });
  const out1 = spec.rows.map(function (r) { return alloc(r * 4); });
  const out2 = spec.rows.map(function (r) { return alloc(r * 4); });
  // (1) the engine's dispatches: one matmulQuant / matmulQ8 / matmulQ4K per matrix, uniform {M: rows, N: n}
  spec.rows.forEach(function (r, i) {
    const u = new Uniform([{ u: r }, { u: spec.n }]);
    if (fmt === 'f16') att.dispatch('matmulQuant', [x, ws[i], out1[i]], u);
    else att.dispatch(fmt === 'q8' ? 'matmulQ8' : 'matmulQ4K', [x, ws[i], metas[i], out1[i]], u);
  });
  // (2) one launch over all of them
  if (fmt === 'f16') {
    att.linear(x, spec.n, spec.rows.map(function (r, i) { return { weight: ws[i], out: out2[i], rows: r }; }));
  } else {
    att.linearQuant(x, spec.n, fmt as 'q8' | 'q4k', spec.rows.map(function (r, i) {
      return { weight: ws[i], meta: metas[i], out: out2[i], rows: r };
    }));
  }
  const total = spec.rows.reduce(function (a, b) { return a + b; }, 0);
  const res = new Uint8Array(2 * total * 4);
  let off = 0;
  for (const outs of [out1, out2]) {
    spec.rows.forEach(function (r, i) {
      att.readBuffer(outs[i], 0, res.subarray(off, off + r * 4));
      off += r * 4;
    });
  }
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return [`engine order: ${spec.rows.length} dispatches`, 'linear: 1 call', 'results written'];
}

interface BatchSpec {
  nqh: number; nkh: number; hd: number; maxBatch: number; maxSeqLen: number; eps: number;
  layers: { slidingWindow: number; theta: number; applyDivisor: number; kvSource: number; headDim: number }[];
  steps: { release: string[]; submit: [string, number][]; admitted: string[] }[];
  arrays: Record<string, number[]>;
}

// Profiled throughout: every token is one forward of the per-pass profiler, whose samples must cover
// every attnStep launch while the outputs stay those the unprofiled path gives (checked by the caller).
async function batch(dir: string): Promise<string[]> {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as BatchSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const bufs: DeviceBuffer[] = [];
  function bytesOf(name: string): Uint8Array {
    const r = spec.arrays[name];
    if (!r) fail(`case.bin has no ${name}`);
    return bin.subarray(r[0], r[0] + r[1]);
  }
  function upload(name: string): DeviceBuffer {
    const data = bytesOf(name);
    const b = att.createBuffer(data.byteLength);
    att.writeBuffer(b, 0, data);
    bufs.push(b);
    return b;
  }
  const rfBytes = bytesOf('rf');
  const rfBits = new Uint16Array(rfBytes.buffer.slice(rfBytes.byteOffset, rfBytes.byteOffset + rfBytes.byteLength));
  const rf = upload('rf');
  const layers = spec.layers.map(function (L, l) {
    return {
      slidingWindow: L.slidingWindow, theta: L.theta, applyDivisor: L.applyDivisor, kvSource: L.kvSource,
      headDim: L.headDim, qWeight: upload('qw' + l), kWeight: upload('kw' + l), ropeFreqs: rf,
      ropeInvFreq: att.ropeInvFreqHost(L.theta, L.headDim, L.applyDivisor, rfBits), eps: spec.eps,
    };
  });
  const sched = new DecodeScheduler(att, {
    shape: { numQHeads: spec.nqh, numKvHeads: spec.nkh, headDim: spec.hd }, layers: layers,
    maxBatch: spec.maxBatch, maxSeqLen: spec.maxSeqLen,
  });
  const outs: Uint8Array[] = [];
  let launches = 0, begins = 0;
  att.enableProfile();
  for (let si = 0; si < spec.steps.length; si++) {
    const st = spec.steps[si];
    st.release.forEach(function (id) { sched.release(id); });
    st.submit.forEach(function (s) { sched.submit(s[0], s[1]); });
    const admitted = sched.admit();
    same(admitted, st.admitted, `step ${si}: admitted`);
    admitted.forEach(function (id) {  // the prompt rows, as prefill would have left them
      spec.layers.forEach(function (L, l) {
        if (L.kvSource !== l) return;
        const kc = bytesOf(`kc:${id}:${l}`), vc = bytesOf(`vc:${id}:${l}`);
        if (kc.byteLength) att.writeBuffer(sched.kCache(id, l), 0, kc);
        if (vc.byteLength) att.writeBuffer(sched.vCache(id, l), 0, vc);
      });
    });
    // steps 0, 4, 8, ... run layer by layer; the others make every layer ready at once (beginToken: a
    // prepare, one upload per head_dim group, or the previous token's plans advanced on the host)
    if (si % 4 !== 0) {
      if (sched.beginToken() !== sched.activeIds().length) fail('beginToken count');
      begins++;
    }
    spec.layers.forEach(function (_L, l) {
      const ids = sched.activeIds();
      const producer = spec.layers[l].kvSource === l;
      ids.forEach(function (id) {  // attn.linearQKV's outputs (attn.linearQ's alone on consumer layers)
        att.writeBuffer(sched.q(id, l), 0, bytesOf(`q:${si}:${id}:${l}`));
        if (!producer) return;
        att.writeBuffer(sched.k(id, l), 0, bytesOf(`k:${si}:${id}:${l}`));
        att.writeBuffer(sched.v(id, l), 0, bytesOf(`v:${si}:${id}:${l}`));
      });
      if (sched.stepLayer(l) !== ids.length) fail('stepLayer count');
      launches++;
      ids.forEach(function (id) {
        const o = sched.out(id, l);
        const host = new Uint8Array(o.size);
        att.readBuffer(o, 0, host);
        outs.push(host);
      });
    });
    sched.advance();
    await att.collectProfileSamples();
  }
  const rep = att.getProfileReport();
  same(rep.forwardSamples_n, spec.steps.length, 'profiled forwards');
  same(rep.perLabel.length, 1, 'profiled labels');
  same(rep.perLabel[0].label, 'attn.decodeFused', 'profiled label');
  same(rep.perLabel[0].samples_n, launches, 'profiled attnStep passes');
  if (!(rep.perLabel[0].p50_ns > 0) || rep.overflow) fail('profile report');
  let total = 0;
  for (const o of outs) total += o.byteLength;
  const res = new Uint8Array(total);
  let off = 0;
  for (const o of outs) {
    res.set(o, off);
    off += o.byteLength;
  }
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  sched.dispose();
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return [`${spec.steps.length} token steps`, `${launches} attnStep launches`, `${outs.length} outputs written`,
    `beginToken: ${sched.prepares} prepared, ${begins - sched.prepares} advanced`,
    `profiled: attn.decodeFused p50 ${(rep.perLabel[0].p50_ns / 1e3).toFixed(1)} us over ${launches} passes`];
}

interface QkvPrepSpec {
  n: number; nqh: number; nkh: number; hd: number; position: number; slot: number; rows: number; theta: number;
  div: number; seq: number; arrays: Record<string, number[]>;
}

// attn.linearQKV with the prep as its epilogue (linearQkvPrep), then the decode step reading the ready q and
// the stored row: out.bin = q, k, v (f32), the cache rows, attnOut.
function qkvPrep(dir: string): string[] {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as QkvPrepSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const bufs: DeviceBuffer[] = [];
  function alloc(bytes: number): DeviceBuffer {
    const b = att.createBuffer(bytes);
    att.clearBuffer(b);
    bufs.push(b);
    return b;
  }
  function upload(name: string): DeviceBuffer {
    const r = spec.arrays[name];
    const b = alloc(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    return b;
  }
  const shape = { numQHeads: spec.nqh, numKvHeads: spec.nkh, headDim: spec.hd };
  const rows = [spec.nqh * spec.hd, spec.nkh * spec.hd, spec.nkh * spec.hd];
  const outs = rows.map(function (r) { return alloc(r * 4); });
  const kc = upload('kc'), vc = upload('vc');
  const segs = rows.map(function (r, i) { return { weight: upload('w' + i), out: outs[i], rows: r }; });
  const qw = upload('qw'), kw = upload('kw'), rf = upload('rf');
  const ws = alloc(att.linearQkvPrepWorkspaceSize(shape));
  att.linearQkvPrep(upload('x'), spec.n, 'f16', segs, {
    qWeight: qw, kWeight: kw, ropeFreqs: rf, kCache: kc, vCache: vc, position: spec.position, slot: spec.slot,
    maxSeqLen: spec.rows, theta: spec.theta, applyDivisor: spec.div,
  }, shape, ws);
  const attnOut = alloc(spec.nqh * spec.hd * 4);
  const stepWs = alloc(att.attnStepWorkspaceSize(1, shape));
  att.attnStep([{ q: outs[0], qWeight: qw, ropeFreqs: rf, kCache: kc, vCache: vc, out: attnOut, seqLen: spec.seq,
    position: spec.position, storeKv: false, theta: spec.theta, applyDivisor: spec.div, qReady: true }], shape, stepWs);
  const parts = [outs[0], outs[1], outs[2], kc, vc, attnOut];
  let total = 0;
  for (const b of parts) total += b.size;
  const res = new Uint8Array(total);
  let off = 0;
  for (const b of parts) {
    att.readBuffer(b, 0, res.subarray(off, off + b.size));
    off += b.size;
  }
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return ['linearQkvPrep: 1 call', 'attnStep (qReady): 1 call', 'results written'];
}

// captureAttention at every per-layer capture point of a KV-producer layer, then postRopeQ and attnOut of a
// consumer layer reading the producer's caches (case.json as qkvPrep's, with `cw0`: the consumer's q
// weight, `cqw`: its q norm); out.bin = the producer's preRopeQ, preRopeK, preRopeV, postRopeQ, postRopeK,
// attnOut, then the consumer's postRopeQ and attnOut (f32), then both caches.
async function capture(dir: string): Promise<string[]> {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'case.json'), 'utf8')) as QkvPrepSpec;
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const att = new HipAttention(loadAddon(), 0);
  const bufs: DeviceBuffer[] = [];
  function alloc(bytes: number): DeviceBuffer {
    const b = att.createBuffer(bytes);
    att.clearBuffer(b);
    bufs.push(b);
    return b;
  }
  function upload(name: string): DeviceBuffer {
    const r = spec.arrays[name];
    const b = alloc(r[1]);
    att.writeBuffer(b, 0, bin.subarray(r[0], r[0] + r[1]));
    return b;
  }
  const shape = { numQHeads: spec.nqh, numKvHeads: spec.nkh, headDim: spec.hd };
  const rows = [spec.nqh * spec.hd, spec.nkh * spec.hd, spec.nkh * spec.hd];
  const kc = upload('kc'), vc = upload('vc'), x = upload('x'), rf = upload('rf');
  const qw = upload('qw'), kw = upload('kw'), cqw = upload('cqw');
  const prepWs = alloc(att.linearQkvPrepWorkspaceSize(shape));
  const stepWs = alloc(att.attnStepWorkspaceSize(1, shape));
  const prep = { ropeFreqs: rf, position: spec.position, slot: spec.slot, maxSeqLen: spec.rows, theta: spec.theta,
    applyDivisor: spec.div };
  const producer = {
    input: x, n: spec.n,
    segments: rows.map(function (r, i) { return { weight: upload('w' + i), out: alloc(r * 4), rows: r }; }),
    prep: Object.assign({ qWeight: qw, kWeight: kw, kCache: kc, vCache: vc }, prep),
    kCache: kc, vCache: vc, seqLen: spec.seq, out: alloc(spec.nqh * spec.hd * 4),
    prepWorkspace: prepWs, stepWorkspace: stepWs,
  };
  const consumer = {
    input: x, n: spec.n, segments: [{ weight: upload('cw0'), out: alloc(rows[0] * 4), rows: rows[0] }],
    prep: Object.assign({ qWeight: cqw }, prep),
    kCache: kc, vCache: vc, seqLen: spec.seq, out: alloc(spec.nqh * spec.hd * 4),
    prepWorkspace: prepWs, stepWorkspace: stepWs,
  };
  const got: Float32Array[] = [];
  for (const k of ['preRopeQ', 'preRopeK', 'preRopeV', 'postRopeQ', 'postRopeK', 'attnOut'] as const) {
    got.push(await att.captureAttention(producer, shape, k));
  }
  got.push(await att.captureAttention(consumer, shape, 'postRopeQ'));
  got.push(await att.captureAttention(consumer, shape, 'attnOut'));
  let refused = '';
  try {
    await att.captureAttention(consumer, shape, 'postRopeK');
  } catch (e) {
    refused = String(e);
  }
  if (refused.indexOf('KV-producer layers only') < 0) fail('postRopeK of a consumer layer not refused: ' + refused);
  let total = kc.size + vc.size;
  for (const g of got) total += g.byteLength;
  const res = new Uint8Array(total);
  let off = 0;
  for (const g of got) {
    res.set(new Uint8Array(g.buffer, g.byteOffset, g.byteLength), off);
    off += g.byteLength;
  }
  att.readBuffer(kc, 0, res.subarray(off, off + kc.size));
  att.readBuffer(vc, 0, res.subarray(off + kc.size, off + kc.size + vc.size));
  fs.writeFileSync(path.join(dir, 'out.bin'), res);
  for (const b of bufs) att.destroyBuffer(b);
  att.dispose();
  return ['captureAttention: 6 points of a producer layer, 2 of a consumer', 'postRopeK of a consumer refused',
    'results written'];
}

// Promise readback: each copy is ordered where it was issued on the stream, whatever enqueues follow it.
function readback(dir: string): Promise<string[]> {
  const bin: Uint8Array = fs.readFileSync(path.join(dir, 'case.bin'));
  const n = bin.byteLength / 4;
  const att = new HipAttention(loadAddon(), 0);
  const b = att.createBuffer(bin.byteLength);
  att.writeBuffer(b, 0, bin);
  att.dispatch('logitSoftcap', [b], new Uniform([{ u: n }, { f: 30.0 }]));
  const first = new Uint8Array(bin.byteLength), second = new Uint8Array(bin.byteLength);
  const p1 = att.readBufferAsync(b, 0, first);  // after the softcap
  att.clearBuffer(b);                           // enqueued after the first copy: not in `first`
  const p2 = att.readBufferAsync(b, 0, second);
  const tooLong = att.readBufferAsync(b, 8, new Uint8Array(bin.byteLength)).then(
    function () { fail('readBufferAsync past the end resolved'); }, function () { return 'range error rejected'; });
  return Promise.all([p1, p2, tooLong]).then(function (r) {
    const res = new Uint8Array(2 * bin.byteLength);
    res.set(first, 0);
    res.set(second, bin.byteLength);
    fs.writeFileSync(path.join(dir, 'out.bin'), res);
    att.destroyBuffer(b);
    att.dispose();
    return ['2 promise readbacks around a clear', r[2] as string, 'results written'];
  });
}

// Per-pass GPU timing (enableProfile / collectProfileSamples / getProfileReport, src/engine.ts:3085-3288):
// labels and sample counts per forward, durations bounded below by the bytes each pass moves at the 8 TB/s
// HBM peak, a forward enqueued while the previous one resolves, the overflow flag, and no timing when off.
async function profile(dir: string): Promise<string[]> {
  const done: string[] = [];
  const att = new HipAttention(loadAddon(), 0);
  const n = 16 << 20;  // 64 MiB of logits: the soft-cap reads and writes 128 MiB
  const big = att.createBuffer(n * 4), small = att.createBuffer(1024);
  att.clearBuffer(big);
  att.clearBuffer(small);
  const capBig = new Uniform([{ u: n }, { f: 30.0 }]), capSmall = new Uniform([{ u: 256 }, { f: 30.0 }]);
  const forward = function () {
    att.dispatch('logitSoftcap', [big], capBig);
    att.dispatch('logitSoftcap', [small], capSmall);
    att.dispatch('logitSoftcap', [big], capBig);
  };
  forward();
  await att.collectProfileSamples();
  same(att.getProfileReport().perLabel.length, 0, 'passes timed while profiling is off');
  att.enableProfile();
  for (let f = 0; f < 3; f++) {
    forward();
    await att.collectProfileSamples();
  }
  forward();
  const p1 = att.collectProfileSamples();
  forward();  // enqueued while the previous forward's timestamps resolve: a set of its own
  const p2 = att.collectProfileSamples();
  await Promise.all([p1, p2]);
  let r = att.getProfileReport();
  same(r.forwardSamples_n, 5, 'forward samples');
  same(r.overflow, false, 'overflow');
  same(r.perLabel.length, 1, 'labels');
  const s = r.perLabel[0];
  same(s.label, 'logitSoftcap', 'label');
  same(s.samples_n, 15, 'samples per label');
  const floor = 2 * n * 4 / 8e12 * 1e9;  // ns for 128 MiB at 8 TB/s
  if (!(s.p50_ns >= floor)) fail(`soft-cap pass p50 ${s.p50_ns} ns under the HBM floor ${floor} ns`);
  if (!(s.p95_ns >= s.p50_ns && s.p95_ns < 5e6)) fail(`soft-cap pass p95 ${s.p95_ns} ns`);
  if (!(r.forwardMedian_ns >= 2 * floor && r.forwardMedian_ns < 2e7)) fail(`forward median ${r.forwardMedian_ns} ns`);
  if (Math.abs(s.total_ns - s.mean_ns * s.samples_n) > 1) fail('total != mean * samples');
  done.push(`5 forwards timed: soft-cap p50 ${(s.p50_ns / 1e3).toFixed(1)} us (HBM floor ${(floor / 1e3).toFixed(1)} us), ` +
    `forward median ${(r.forwardMedian_ns / 1e3).toFixed(1)} us`);
  // more passes than the set holds: the excess runs untimed and the report says so
  att.resetProfileSamples();
  const slots = att.getProfileCapability().querySlots;
  for (let i = 0; i < slots / 2 + 5; i++) att.dispatch('logitSoftcap', [small], capSmall);
  await att.collectProfileSamples();
  r = att.getProfileReport();
  same(r.overflow, true, 'overflow after too many passes');
  same(r.perLabel[0].samples_n <= slots / 2, true, 'samples within the set');
  done.push(`overflow flagged after ${slots / 2 + 5} passes (${r.perLabel[0].samples_n} timed)`);
  att.resetProfileSamples();
  att.disableProfile();
  forward();
  await att.collectProfileSamples();
  same(att.getProfileReport().perLabel.length, 0, 'passes timed after disableProfile');
  done.push('no timing when off');
  att.destroyBuffer(big);
  att.destroyBuffer(small);
  att.dispose();
  return done;
}

export function main(argv: string[]): void {
  const mode = argv[0];
  if (mode === 'readback' || mode === 'profile' || mode === 'batch' || mode === 'capture') {
    (mode === 'readback' ? readback(argv[1]) : mode === 'profile' ? profile(argv[1])
      : mode === 'capture' ? capture(argv[1]) : batch(argv[1])).then(function (done) {
      process.stdout.write(JSON.stringify({ ok: true, checks: done }) + '\n');
    }, function (e) {
      process.stderr.write(String(e && e.stack ? e.stack : e) + '\n');
      process.exitCode = 1;
    });
    return;
  }
  let done: string[];
  if (mode === 'cpu') done = cpuChecks();
  else if (mode === 'layer') done = layer(argv[1]);
  else if (mode === 'head') done = head(argv[1]);
  else if (mode === 'prefill') done = prefill(argv[1]);
  else if (mode === 'promptprep') done = promptPrep(argv[1]);
  else if (mode === 'linear') done = linear(argv[1]);
  else if (mode === 'qkvprep') done = qkvPrep(argv[1]);
  else fail(`usage: run.js cpu | layer <dir> | prefill <dir> | promptprep <dir> | head <dir> | linear <dir> | qkvprep <dir> | capture <dir> | batch <dir> | readback <dir> | profile`);
  process.stdout.write(JSON.stringify({ ok: true, checks: done }) + '\n');
}
