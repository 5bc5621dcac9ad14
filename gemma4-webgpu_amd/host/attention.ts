// Host side of the gfx950 attention path: the engine's attention dispatch
// surface (src/shaders.ts:43-74 names, src/engine.ts:2056-2094 call order),
// served by libg4attn.so through the g4attn.node N-API addon.
//
// - Kernel names are the engine's SHADERS keys; bindings are passed in the
//   WGSL @binding order of each shader; Params are the same uniform bytes the
//   engine builds with makeUniformMixed (src/engine.ts:460-478) and patches
//   per token with wb() (src/engine.ts:1967-1987), passed by value at enqueue
//   time, so a later patch never affects work already enqueued.
// - The backend is chosen once, at construction; no call falls back to
//   anything else. Every library error is thrown as an Error with the
//   library's message.
// - attnStep is the fused replacement of the six dispatches for any number of
//   layers or sequences (one attention launch plus one merge launch).

declare const require: any;
declare const __dirname: string;

export type AttnKernelName =
  | 'fusedPerHeadNormRope'
  | 'perHeadRmsNormNoWeight'
  | 'kvCacheStore'
  | 'attnScore'
  | 'softmax'
  | 'attnOutput';

// The sampling head after the last layer (src/engine.ts:2223-2255).
export type SampleKernelName = 'matmulQuant' | 'logitSoftcap' | 'argmax';

// The in-shader quantized GEMVs of the block's projections (weightQuant 'q8' / 'q4k', src/engine.ts:2040-2043).
export type QuantKernelName = 'matmulQ8' | 'matmulQ4K';

export type KernelName = AttnKernelName | SampleKernelName | QuantKernelName;

export type FusedKernelName = 'attnStep' | 'attnPrefill' | 'attnPromptPrep' | 'lmHeadArgmax' | 'linearQkvPrep';

export type UniformValue = { u: number } | { f: number };

// Storage bindings of each kernel in @binding order (the uniform is separate).
export const BINDINGS: Record<KernelName, string[]> = {
  fusedPerHeadNormRope: ['data', 'weight', 'rope_freqs'],  // fused_per_head_norm_rope.wgsl:14-17
  perHeadRmsNormNoWeight: ['data'],                          // per_head_rms_norm_no_weight.wgsl:9
  kvCacheStore: ['k_in', 'v_in', 'k_cache', 'v_cache'],     // kv_cache_store.wgsl:2-5
  attnScore: ['q', 'k_cache', 'scores'],                     // attn_score.wgsl:10-12
  softmax: ['scores'],                                       // softmax.wgsl:2
  attnOutput: ['probs', 'v_cache', 'output'],                // attn_output.wgsl:2-4
  matmulQuant: ['input', 'weight', 'output'],                // matmul_quant.wgsl:13-15 (f16 weight)
  logitSoftcap: ['logits'],                                  // logit_softcap.wgsl:6
  argmax: ['logits', 'result'],                              // argmax.wgsl:1-2
  matmulQ8: ['input', 'qweight', 'qscale', 'output'],        // matmul_q8.wgsl:16-19
  matmulQ4K: ['input', 'qweight', 'qmeta', 'output'],        // matmul_q4k.wgsl:20-23
};

// Params byte sizes (struct Params of each shader).
export const PARAMS_BYTES: Record<KernelName, number> = {
  fusedPerHeadNormRope: 24,
  perHeadRmsNormNoWeight: 16,
  kvCacheStore: 16,
  attnScore: 24,
  softmax: 8,
  attnOutput: 16,
  matmulQuant: 8,
  logitSoftcap: 8,
  argmax: 4,
  matmulQ8: 8,
  matmulQ4K: 8,
};

// Profiler pass labels of the engine (src/engine.ts:2056-2094), plus the fused step.
export const PASS_LABELS: Record<string, string> = {
  perHeadRmsNormNoWeight: 'attn.vNorm',
  fusedPerHeadNormRope: 'attn.fusedNormRopeQK',
  kvCacheStore: 'attn.kvCacheStore',
  attnScore: 'attn.attnScore',
  softmax: 'attn.softmax',
  attnOutput: 'attn.attnOutput',
  attnStep: 'attn.decodeFused',
  attnPrefill: 'attn.prefill',
  attnPromptPrep: 'attn.promptPrep',
  matmulQuant: 'lmHead',
  logitSoftcap: 'logitSoftcap',
  argmax: 'sample.argmax',
  lmHeadArgmax: 'sample.lmHeadArgmax',
  matmulQ8: 'attn.linearQKV',
  matmulQ4K: 'attn.linearQKV',
  linear: 'attn.linearQKV',
  linearOut: 'attn.linearOut',
  attnStepOut: 'attn.linearOut',
  linearQkvPrep: 'attn.linearQKVPrep',
};

// The profiler's report types (src/types.ts:490-515).
export interface ProfileCapability {
  timestampQuerySupported: boolean;
  timestampQueryOnAdapterButUnrequested: boolean;
  querySlots: number;
}

export interface ProfileReport {
  perLabel: Array<{ label: string; samples_n: number; p50_ns: number; p95_ns: number; mean_ns: number; total_ns: number }>;
  forwardMedian_ns: number;
  forwardSamples_n: number;
  overflow: boolean;
}

// The engine's makeUniformMixed: 4-byte fields, at least 16 bytes.
export class Uniform {
  readonly bytes: Uint8Array;
  private readonly u32: Uint32Array;
  private readonly f32: Float32Array;

  constructor(values: UniformValue[]) {
    const size = Math.max(values.length * 4, 16);
    const ab = new ArrayBuffer(size);
    this.u32 = new Uint32Array(ab);
    this.f32 = new Float32Array(ab);
    this.bytes = new Uint8Array(ab);
    for (let i = 0; i < values.length; i++) {
      const v = values[i];
      if ('u' in v) this.u32[i] = v.u;
      else this.f32[i] = v.f;
    }
  }

  // The engine's wb(buffer, byteOffset, u32Value) per-token patch.
  writeU32(byteOffset: number, value: number): void {
    this.u32[byteOffset >> 2] = value >>> 0;
  }

  writeF32(byteOffset: number, value: number): void {
    this.f32[byteOffset >> 2] = value;
  }
}

export interface DeviceBuffer {
  readonly ptr: bigint;
  readonly size: number;
}

// One entry of the fused step: a layer of a token's stack or a sequence of a batch.
export interface StepEntry {
  q: DeviceBuffer;            // raw projection f32 [NQH][HD] (read only)
  k?: DeviceBuffer;           // raw projection f32 [NKH][HD]; k, v and kWeight absent (with storeKv false):
  v?: DeviceBuffer;           // the current row is already in the cache (a consumer layer after its producer)
  qWeight: DeviceBuffer;      // attn_q_norm f16 [HD]
  kWeight?: DeviceBuffer;     // attn_k_norm f16 [HD]
  ropeFreqs?: DeviceBuffer;   // f16 divisor table (global layers)
  ropeInvFreq?: Float32Array; // host f32 [HD/2] table from ropeInvFreqHost(); RoPE factors are then evaluated in prepare
  kCache: DeviceBuffer;       // f16 [rows][NKH][HD]
  vCache: DeviceBuffer;
  out: DeviceBuffer;          // attnOut f32 [NQH][HD]
  seqLen: number;             // rows including the current token's (row seqLen - 1)
  position: number;           // RoPE position
  slidingWindow?: number;     // 0 = full
  storeKv?: boolean;          // false on KV-consumer layers
  theta: number;
  applyDivisor?: number;
  scale?: number;
  eps?: number;
  qReady?: boolean;           // q already holds the post-norm, post-RoPE query (linearQkvPrep's output)
}

// One prefill entry: a chunk of tokens of one layer (or sequence). Token t sits at position start + t and
// attends cache rows [lo, start + t] (lo = start + t + 1 - slidingWindow on local layers, else 0), the rows
// the decode step at that position reads. The caches already hold the chunk's own K/V rows.
export interface PrefillEntry {
  q: DeviceBuffer;            // post norm + RoPE queries, f16 [nTokens][NQH][HD]
  kCache: DeviceBuffer;       // f16 [rows >= start + nTokens][NKH][HD]
  vCache: DeviceBuffer;
  out: DeviceBuffer;          // f32 [nTokens][NQH][HD]
  nTokens: number;
  start: number;
  slidingWindow?: number;     // 0 = full
  scale?: number;
  vtCache?: DeviceBuffer;     // V^T blocks of vCache written by attnPromptPrep (PromptPrep.vtCache), holding
  vtRows?: number;            // every attended row; vtRows: the maxSeqLen it was sized for
}

// The prep of a prompt chunk of one layer (the engine's per-token vNorm -> fusedNormRope(Q, K) ->
// kvCacheStore, src/engine.ts:2460-2479, for every token at once). Token t sits at position start + t.
export interface PromptPrep {
  q: DeviceBuffer;            // raw projections f32 [nTokens][NQH][HD] (read only)
  k?: DeviceBuffer;           // f32 [nTokens][NKH][HD]; k, v, kWeight and the caches absent on KV-consumer
  v?: DeviceBuffer;           // layers (only q is prepared)
  qWeight: DeviceBuffer;      // attn_q_norm f16 [HD]
  kWeight?: DeviceBuffer;     // attn_k_norm f16 [HD]
  ropeFreqs?: DeviceBuffer;   // f16 divisor table (global layers)
  ropeInvFreq?: DeviceBuffer; // f32 [HD/2] from ropeInvFreq for this layer's theta/divisor (computed once, at load)
  qOut: DeviceBuffer;         // f16 [nTokens][NQH][HD]: PrefillEntry.q
  kCache?: DeviceBuffer;      // f16 [maxSeqLen][NKH][HD]: rows start .. start + nTokens - 1 are written
  vCache?: DeviceBuffer;
  vtCache?: DeviceBuffer;     // producer layers, optional: the V rows also as V^T blocks
                              // f16 [NKH][ceil(maxSeqLen / 32)][HD][32], which attnPrefill reads V from
  nTokens: number;
  start: number;
  theta: number;
  applyDivisor: number;
  maxSeqLen?: number;
  eps?: number;
}

// linearQkvPrep: one segment of the q/k/v projection (q, then k and v on producer layers).
export interface QkvSegment {
  weight: DeviceBuffer;       // f16 [rows][n], int8 [rows][n] (q8) or u32 [rows][n/8] (q4k)
  meta?: DeviceBuffer;        // q8 / q4k scales (as linearQuant)
  out: DeviceBuffer;          // f32 [rows]: the layer's q / k / v buffer
  rows: number;
}

// linearQkvPrep's epilogue: the layer's norms, RoPE configuration and, on producer layers, the cache row.
export interface QkvPrep {
  qWeight: DeviceBuffer;      // attn_q_norm f16 [HD]
  kWeight?: DeviceBuffer;     // attn_k_norm f16 [HD] (producer layers)
  ropeFreqs?: DeviceBuffer;   // f16 divisor table (global layers)
  ropeInvFreq?: DeviceBuffer; // f32 [HD/2] from ropeInvFreq (computed once, at load)
  kCache?: DeviceBuffer;      // f16 [maxSeqLen][NKH][HD]: row `slot` is written (producer layers)
  vCache?: DeviceBuffer;
  position: number;
  slot?: number;
  maxSeqLen?: number;
  theta: number;
  applyDivisor?: number;
  eps?: number;
}

// captureHidden's per-layer capture points (src/engine.ts:2749-2815; the kinds of src/types.ts:341-348):
// after the q/k/v projection, after the per-head norms and RoPE, after the attention.
export type AttnCapturePoint = 'preRopeQ' | 'preRopeK' | 'preRopeV' | 'postRopeQ' | 'postRopeK' | 'attnOut';

// One layer's attention block for one token, as captureAttention runs it.
export interface AttnCaptureLayer {
  input: DeviceBuffer;        // the attention-normed hidden state f32 [n]
  n: number;
  segments: QkvSegment[];     // f16 weights: q, then k and v on KV-producer layers (outs: the layer's q/k/v)
  prep: QkvPrep;              // norms, RoPE and (producer layers) the cache row at `slot` = seqLen - 1
  kCache: DeviceBuffer;       // the caches the layer attends (its producer's on a consumer layer)
  vCache: DeviceBuffer;
  seqLen: number;
  slidingWindow?: number;
  scale?: number;
  out: DeviceBuffer;          // attnOut f32 [NQH][HD]
  prepWorkspace: DeviceBuffer;  // linearQkvPrepWorkspaceSize bytes, cleared once
  stepWorkspace: DeviceBuffer;  // attnStepWorkspaceSize(1) bytes
}

// The fused sampling head: lm head over an f16 [vocab][hidden] weight, softcap (0 = none), argmax.
export interface LmHeadShape {
  vocab: number;
  hidden: number;
  cap: number;
}

// One f16 weight matrix of a projection: out[r] = sum_c weight[r][c] * input[c] (matmulQuant's rows).
export interface LinearSegment {
  weight: DeviceBuffer;       // f16 [rows][n]
  out: DeviceBuffer;          // f32 [rows]
  rows: number;
}

// One quantized weight matrix: q8 (int8 [rows][n] + f16 scales [rows][n/32]) or q4k (u32 [rows][n/8] +
// f16 meta [rows][n/256][16]: 8 scales then 8 mins per 256-element super-block).
export interface QuantSegment {
  weight: DeviceBuffer;
  meta: DeviceBuffer;
  out: DeviceBuffer;          // f32 [rows]
  rows: number;
}

export interface StepShape {
  numQHeads: number;
  numKvHeads: number;
  headDim: number;
}

// What g4attn.node exports (gemma4-webgpu_amd/addon/g4attn_napi.cc).
export interface Addon {
  version(): string;
  deviceCount(): number;
  setDevice(d: number): void;
  streamCreate(): bigint;
  streamDestroy(s: bigint): void;
  streamSynchronize(s: bigint): void;
  malloc(bytes: number): bigint;
  free(p: bigint): void;
  upload(dst: bigint, offset: number, data: any, s: bigint): void;
  download(src: bigint, offset: number, out: any, s: bigint): void;
  readAsync(src: bigint, offset: number, out: any, s: bigint): Promise<void>;
  querySetCreate(count: number): bigint;
  queryBeginPass(set: bigint, slot: number): void;
  queryEndPass(): void;
  queryWrite(set: bigint, slot: number, s: bigint): void;
  queryResolve(set: bigint, first: number, nPairs: number): Float64Array;
  queryResolveAsync(set: bigint, first: number, nPairs: number): Promise<Float64Array>;
  querySetDestroy(set: bigint): void;
  zero(p: bigint, bytes: number, s: bigint): void;
  fusedPerHeadNormRope(data: bigint, w: bigint, rf: bigint, p: Uint8Array, s: bigint): void;
  perHeadRmsNormNoWeight(data: bigint, p: Uint8Array, s: bigint): void;
  kvCacheStore(k: bigint, v: bigint, kc: bigint, vc: bigint, p: Uint8Array, s: bigint): void;
  attnScore(q: bigint, kc: bigint, sc: bigint, p: Uint8Array, s: bigint): void;
  softmax(sc: bigint, p: Uint8Array, s: bigint): void;
  attnOutput(pr: bigint, vc: bigint, o: bigint, p: Uint8Array, s: bigint): void;
  matmulQuant(x: bigint, w: bigint, o: bigint, p: Uint8Array, s: bigint): void;
  matmulQ8(x: bigint, q: bigint, sc: bigint, o: bigint, p: Uint8Array, s: bigint): void;
  matmulQ4K(x: bigint, q: bigint, m: bigint, o: bigint, p: Uint8Array, s: bigint): void;
  linearQuant(x: bigint, n: number, format: number, segs: { weight: bigint; meta: bigint; out: bigint; rows: number }[],
    s: bigint): void;
  linearQkvPrepWorkspaceSize(nqh: number, nkh: number): number;
  linearQkvPrep(x: bigint, n: number, format: number, segs: { weight: bigint; meta?: bigint; out: bigint; rows: number }[],
    qw: bigint, kw: bigint | null, rf: bigint | null, inv: bigint | null, kc: bigint | null, vc: bigint | null,
    p: Uint8Array, ws: bigint, s: bigint): void;
  logitSoftcap(l: bigint, p: Uint8Array, s: bigint): void;
  argmax(l: bigint, r: bigint, p: Uint8Array, s: bigint): void;
  lmHeadWorkspaceSize(vocab: number, hidden: number, cap: number): number;
  lmHeadArgmax(h: bigint, w: bigint, l: bigint | null, r: bigint, ws: bigint, wsBytes: number, vocab: number,
    hidden: number, cap: number, s: bigint): void;
  linear(x: bigint, n: number, segs: { weight: bigint; out: bigint; rows: number }[], s: bigint): void;
  ropeInvFreq(theta: number, hd: number, div: number, rf: any, out: bigint, s: bigint): void;
  ropeInvFreqHost(theta: number, hd: number, div: number, rf: Uint16Array | null, out: Float32Array): void;
  attnStepWorkspaceSize(n: number, nqh: number, nkh: number, hd: number): number;
  attnStepPrepare(entries: any[], nqh: number, nkh: number, hd: number, ws: bigint, wsBytes: number,
    s: bigint): Uint8Array;
  attnStepLayersWorkspaceSize(n: number, perLayer: number, nqh: number, nkh: number, hd: number): number;
  attnStepPrepareLayers(entries: any[], perLayer: number, nqh: number, nkh: number, hd: number, ws: bigint,
    wsBytes: number, s: bigint): Uint8Array[];
  attnStepRun(plan: Uint8Array, s: bigint): void;
  attnStepRunPair(plan1: Uint8Array, plan2: Uint8Array, s: bigint): void;
  attnStepAdvance(plan: Uint8Array, tokens: number): void;
  attnStepRunAttention(plan: Uint8Array, s: bigint): void;
  attnStepRunOut(plan: Uint8Array, segs: { weight: bigint; out: bigint; rows: number }[], s: bigint): void;
  attnPrefillWorkspaceSize(entries: any[], nqh: number, nkh: number, hd: number): number;
  attnPrefillPrepare(entries: any[], nqh: number, nkh: number, hd: number, ws: bigint, wsBytes: number,
    s: bigint): Uint8Array;
  attnPrefillRun(plan: Uint8Array, s: bigint): void;
  attnPromptPrep(q: bigint, k: bigint | null, v: bigint | null, qw: bigint, kw: bigint | null, rf: bigint | null,
    inv: bigint | null, qOut: bigint, kc: bigint | null, vc: bigint | null, p: Uint8Array, s: bigint): void;
  attnPromptPrepVt(q: bigint, k: bigint, v: bigint, qw: bigint, kw: bigint, rf: bigint | null,
    inv: bigint | null, qOut: bigint, kc: bigint, vc: bigint, vt: bigint, p: Uint8Array, s: bigint): void;
  attnPromptPrepMany(entries: Uint8Array, n: number, s: bigint): void;
  [key: string]: any;
}

export function loadAddon(path?: string): Addon {
  const p = path || require('path').join(__dirname, '..', 'lib', 'g4attn.node');
  return require(p) as Addon;
}

// The kernel table: SHADERS name -> launch with (bindings in @binding order, Params bytes).
type Launch = (g4: Addon, b: bigint[], p: Uint8Array, s: bigint) => void;
export const KERNELS: Record<KernelName, Launch> = {
  fusedPerHeadNormRope: function (g4, b, p, s) { g4.fusedPerHeadNormRope(b[0], b[1], b[2], p, s); },
  perHeadRmsNormNoWeight: function (g4, b, p, s) { g4.perHeadRmsNormNoWeight(b[0], p, s); },
  kvCacheStore: function (g4, b, p, s) { g4.kvCacheStore(b[0], b[1], b[2], b[3], p, s); },
  attnScore: function (g4, b, p, s) { g4.attnScore(b[0], b[1], b[2], p, s); },
  softmax: function (g4, b, p, s) { g4.softmax(b[0], p, s); },
  attnOutput: function (g4, b, p, s) { g4.attnOutput(b[0], b[1], b[2], p, s); },
  matmulQuant: function (g4, b, p, s) { g4.matmulQuant(b[0], b[1], b[2], p, s); },
  logitSoftcap: function (g4, b, p, s) { g4.logitSoftcap(b[0], p, s); },
  argmax: function (g4, b, p, s) { g4.argmax(b[0], b[1], p, s); },
  matmulQ8: function (g4, b, p, s) { g4.matmulQ8(b[0], b[1], b[2], b[3], p, s); },
  matmulQ4K: function (g4, b, p, s) { g4.matmulQ4K(b[0], b[1], b[2], b[3], p, s); },
};

// Query slots per forward (the engine's PROFILE_QUERY_SLOTS, src/engine.ts:148): two per timed pass.
export const PROFILE_QUERY_SLOTS = 2048;

// The timing behind the profiler API. A forward (the passes enqueued between two harvests) owns one
// query set and takes two slots of it per pass, in pass order. harvest() closes the forward and resolves
// its set off the JS thread; the next pass opens a new forward on a spare set (or a new one), so the
// passes enqueued while a resolve runs never re-record the events it reads. Durations accumulate per
// label, and each forward's sum of durations is kept for the forward median. A pass that finds its
// forward's set full runs untimed and the report says so.
class PassTimer {
  on = false;
  private readonly g4: Addon;
  private current: { set: bigint; labels: string[] } | null = null;  // the open forward
  private readonly spares: bigint[] = [];
  private readonly durations: Map<string, number[]> = new Map();
  private readonly forwardSums: number[] = [];
  private full = false;
  private gone = false;

  constructor(g4: Addon) {
    this.g4 = g4;
  }

  begin(label: string): number {
    if (!this.on) return -1;
    if (this.current === null) {
      const set = this.spares.length ? this.spares.pop() as bigint : this.g4.querySetCreate(PROFILE_QUERY_SLOTS);
      this.current = { set: set, labels: [] };
    }
    const first = 2 * this.current.labels.length;
    if (first + 2 > PROFILE_QUERY_SLOTS) {
      this.full = true;
      return -1;
    }
    this.g4.queryBeginPass(this.current.set, first);
    this.current.labels.push(label);
    return first;
  }

  harvest(): Promise<void> {
    const fwd = this.current;
    this.current = null;
    if (fwd === null) return Promise.resolve();
    const timer = this;
    const recycle = function () {
      if (timer.gone) timer.g4.querySetDestroy(fwd.set);
      else timer.spares.push(fwd.set);
    };
    return this.g4.queryResolveAsync(fwd.set, 0, fwd.labels.length).then(function (ns: Float64Array) {
      recycle();
      let sum = 0;
      fwd.labels.forEach(function (label, i) {
        const d = ns[i];
        if (!(d > 0)) return;  // NaN: the pass launched no kernel
        sum += d;
        const list = timer.durations.get(label);
        if (list) list.push(d);
        else timer.durations.set(label, [d]);
      });
      if (sum > 0) timer.forwardSums.push(sum);
    }, function (e: any) {
      recycle();
      throw e;
    });
  }

  clear(): void {
    this.durations.clear();
    this.forwardSums.length = 0;
    this.full = false;
  }

  report(): ProfileReport {
    // the sample at rank floor(n f) of the sorted samples (the last one at most)
    function rank(sorted: number[], f: number): number {
      return sorted[Math.min(sorted.length - 1, Math.floor(sorted.length * f))];
    }
    function ascending(a: number, b: number): number { return a - b; }
    const rows: ProfileReport['perLabel'] = [];
    this.durations.forEach(function (list, label) {
      if (!list.length) return;
      const sorted = list.slice().sort(ascending);
      const total = list.reduce(function (acc, x) { return acc + x; }, 0);
      rows.push({ label: label, samples_n: list.length, p50_ns: rank(sorted, 0.5), p95_ns: rank(sorted, 0.95),
        mean_ns: total / list.length, total_ns: total });
    });
    rows.sort(function (a, b) { return b.p50_ns - a.p50_ns; });
    const sums = this.forwardSums.slice().sort(ascending);
    return { perLabel: rows, forwardMedian_ns: sums.length ? rank(sums, 0.5) : 0, forwardSamples_n: sums.length,
      overflow: this.full };
  }

  // After the stream is drained: every set this timer holds is destroyed (one still being resolved is
  // destroyed when its resolve ends).
  destroy(): void {
    this.gone = true;
    if (this.current !== null) this.g4.querySetDestroy(this.current.set);
    this.current = null;
    for (const set of this.spares) this.g4.querySetDestroy(set);
    this.spares.length = 0;
  }
}

export class HipAttention {
  readonly stream: bigint;
  private readonly g4: Addon;
  private alive: boolean;
  private readonly timer: PassTimer;  // per-pass GPU timing (the engine's profiler API, below)

  constructor(addon: Addon, device: number) {
    this.g4 = addon;
    addon.setDevice(device);
    this.stream = addon.streamCreate();
    this.alive = true;
    this.timer = new PassTimer(addon);
  }

  version(): string {
    return this.g4.version();
  }

  createBuffer(size: number): DeviceBuffer {
    return { ptr: this.g4.malloc(size), size: size };
  }

  destroyBuffer(b: DeviceBuffer): void {
    this.g4.free(b.ptr);
  }

  writeBuffer(b: DeviceBuffer, offset: number, data: ArrayBufferView): void {
    if (offset + data.byteLength > b.size) throw new RangeError(`writeBuffer: ${offset}+${data.byteLength} > ${b.size}`);
    this.g4.upload(b.ptr, offset, data, this.stream);
  }

  // Blocking read (the engine's mapAsync readback, made synchronous).
  readBuffer(b: DeviceBuffer, offset: number, out: ArrayBufferView): void {
    if (offset + out.byteLength > b.size) throw new RangeError(`readBuffer: ${offset}+${out.byteLength} > ${b.size}`);
    this.g4.download(b.ptr, offset, out, this.stream);
  }

  // mapAsync's shape: the copy is ordered on the stream now (after the work already enqueued, before
  // anything enqueued later); the promise resolves once `out` holds the bytes. The wait runs off the
  // JS thread.
  readBufferAsync(b: DeviceBuffer, offset: number, out: ArrayBufferView): Promise<void> {
    if (offset + out.byteLength > b.size) {
      return Promise.reject(new RangeError(`readBufferAsync: ${offset}+${out.byteLength} > ${b.size}`));
    }
    return this.g4.readAsync(b.ptr, offset, out, this.stream);
  }

  clearBuffer(b: DeviceBuffer): void {
    this.g4.zero(b.ptr, b.size, this.stream);
  }

  // setPipeline(name) + setBindGroup(bindings, params) + dispatchWorkgroups, as one enqueue.
  dispatch(name: KernelName, bindings: DeviceBuffer[], params: Uniform): void {
    const launch = KERNELS[name];
    if (!launch) throw new Error(`unknown kernel ${name}`);
    const want = BINDINGS[name];
    if (bindings.length !== want.length) {
      throw new Error(`${name}: ${bindings.length} bindings, expected ${want.length} (${want.join(', ')})`);
    }
    if (params.bytes.byteLength < PARAMS_BYTES[name]) throw new Error(`${name}: params too short`);
    const slot = this.beginPass(PASS_LABELS[name]);
    try {
      launch(this.g4, bindings.map(function (b) { return b.ptr; }), params.bytes, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  ropeInvFreq(theta: number, headDim: number, applyDivisor: number, ropeFreqs: DeviceBuffer | null,
    out: DeviceBuffer): void {
    this.g4.ropeInvFreq(theta, headDim, applyDivisor, ropeFreqs ? ropeFreqs.ptr : null, out.ptr, this.stream);
  }

  // The same table on the host, for StepEntry.ropeInvFreq; ropeFreqsBits: the f16 bits of the divisor table.
  ropeInvFreqHost(theta: number, headDim: number, applyDivisor: number, ropeFreqsBits: Uint16Array | null): Float32Array {
    const out = new Float32Array(headDim / 2);
    this.g4.ropeInvFreqHost(theta, headDim, applyDivisor, ropeFreqsBits, out);
    return out;
  }

  attnStepWorkspaceSize(nEntries: number, shape: StepShape): number {
    return this.g4.attnStepWorkspaceSize(nEntries, shape.numQHeads, shape.numKvHeads, shape.headDim);
  }

  // Prepare once per token (the entries' seqLen/position change); run as often as wanted.
  attnStepPrepare(entries: StepEntry[], shape: StepShape, workspace: DeviceBuffer): Uint8Array {
    return this.g4.attnStepPrepare(HipAttention.stepFlat(entries), shape.numQHeads, shape.numKvHeads,
      shape.headDim, workspace.ptr, workspace.size, this.stream);
  }

  attnStepLayersWorkspaceSize(nLayers: number, shape: StepShape, entriesPerLayer?: number): number {
    return this.g4.attnStepLayersWorkspaceSize(nLayers, entriesPerLayer || 1, shape.numQHeads, shape.numKvHeads,
      shape.headDim);
  }

  // One token's layers in the engine's order (src/engine.ts:2029-2156), prepared together once per token
  // (where the engine patches every layer's uniforms, :1967-1987) with one table upload: layer i is
  // entries[i * entriesPerLayer ..) (one per layer for a single sequence, the active batch for a batched
  // decode); a plan per layer, each run on its own, in layer order (attnStepRun, or attnStepRunAttention
  // then attnStepOut).
  attnStepPrepareLayers(entries: StepEntry[], shape: StepShape, workspace: DeviceBuffer,
    entriesPerLayer?: number): Uint8Array[] {
    return this.g4.attnStepPrepareLayers(HipAttention.stepFlat(entries), entriesPerLayer || 1, shape.numQHeads,
      shape.numKvHeads, shape.headDim, workspace.ptr, workspace.size, this.stream);
  }

  private static stepFlat(entries: StepEntry[]): any[] {
    return entries.map(function (e) {
      return {
        q: e.q.ptr, k: e.k ? e.k.ptr : undefined, v: e.v ? e.v.ptr : undefined, qWeight: e.qWeight.ptr,
        kWeight: e.kWeight ? e.kWeight.ptr : undefined,
        ropeFreqs: e.ropeFreqs ? e.ropeFreqs.ptr : undefined,
        ropeInvFreq: e.ropeInvFreq,
        kCache: e.kCache.ptr, vCache: e.vCache.ptr, out: e.out.ptr,
        seqLen: e.seqLen, position: e.position, slidingWindow: e.slidingWindow || 0,
        storeKv: e.storeKv === undefined ? true : e.storeKv, theta: e.theta, applyDivisor: e.applyDivisor || 0,
        scale: e.scale === undefined ? 1.0 : e.scale, eps: e.eps === undefined ? 1e-6 : e.eps,
        qReady: e.qReady ? 1 : 0,
      };
    });
  }

  attnStepRun(plan: Uint8Array): void {
    const slot = this.beginPass(PASS_LABELS.attnStep);
    try {
      this.g4.attnStepRun(plan, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  // A token of a model with two head_dims (E2B: 512 on the global layers, 256 on the local ones), one plan
  // per head_dim (either order): both attention passes in one launch, the head_dim-256 workgroups in the
  // tail of the head_dim-512 ones, then both merges in one launch.
  attnStepRunPair(plan1: Uint8Array, plan2: Uint8Array): void {
    const slot = this.beginPass(PASS_LABELS.attnStep);
    try {
      this.g4.attnStepRunPair(plan1, plan2, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  // The next token(s) of a prepared plan without a new prepare: every entry's seqLen and position grow by
  // `tokens` (the engine's per-token uniform patch, src/engine.ts:1967-1987), in place, on the host alone
  // (nothing is enqueued); the kernel evaluates the new positions' RoPE factors. Prepare again every few
  // dozen tokens (the part holding a full layer's last row takes the new rows) and whenever the entries
  // change otherwise; throws past 4096 tokens since the prepare.
  attnStepAdvance(plan: Uint8Array, tokens?: number): void {
    this.g4.attnStepAdvance(plan, tokens === undefined ? 1 : tokens);
  }

  attnStep(entries: StepEntry[], shape: StepShape, workspace: DeviceBuffer): void {
    this.attnStepRun(this.attnStepPrepare(entries, shape, workspace));
  }

  // The attention pass of a prepared step alone; attnStepOut then finishes it.
  attnStepRunAttention(plan: Uint8Array): void {
    const slot = this.beginPass(PASS_LABELS.attnStep);
    try {
      this.g4.attnStepRunAttention(plan, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  // attn.linearOut of every entry of a step after attnStepRunAttention (src/engine.ts:2096), with the step's
  // merge folded into the projection's launch: each entry's attnOut is written as attnStepRun writes it, and
  // segments[i].out = segments[i].weight (f16 [rows][numQHeads * headDim]) x attnOut, each row bit-identical
  // to linear() over that attnOut. One segment per entry, in entry order.
  attnStepOut(plan: Uint8Array, shape: StepShape, segments: LinearSegment[]): void {
    const n = shape.numQHeads * shape.headDim;
    const segs = segments.map(function (g, i) {
      if (g.weight.size < g.rows * n * 2) throw new RangeError('attnStepOut: segment ' + i + ' weight too small');
      if (g.out.size < g.rows * 4) throw new RangeError('attnStepOut: segment ' + i + ' out too small');
      return { weight: g.weight.ptr, out: g.out.ptr, rows: g.rows };
    });
    const slot = this.beginPass(PASS_LABELS.attnStepOut);
    try {
      this.g4.attnStepRunOut(plan, segs, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  private static prefillFlat(entries: PrefillEntry[]): any[] {
    return entries.map(function (e) {
      return {
        q: e.q.ptr, kCache: e.kCache.ptr, vCache: e.vCache.ptr, out: e.out.ptr, nTokens: e.nTokens,
        start: e.start, slidingWindow: e.slidingWindow || 0, scale: e.scale === undefined ? 1.0 : e.scale,
        vtCache: e.vtCache ? e.vtCache.ptr : undefined, vtRows: e.vtRows || 0,
      };
    });
  }

  attnPrefillWorkspaceSize(entries: PrefillEntry[], shape: StepShape): number {
    return this.g4.attnPrefillWorkspaceSize(HipAttention.prefillFlat(entries), shape.numQHeads, shape.numKvHeads,
      shape.headDim);
  }

  // Prepare once per set of chunks; run as often as wanted (one attention launch, plus a merge when a
  // chunk's key range was split).
  attnPrefillPrepare(entries: PrefillEntry[], shape: StepShape, workspace: DeviceBuffer): Uint8Array {
    return this.g4.attnPrefillPrepare(HipAttention.prefillFlat(entries), shape.numQHeads, shape.numKvHeads,
      shape.headDim, workspace.ptr, workspace.size, this.stream);
  }

  attnPrefillRun(plan: Uint8Array): void {
    const slot = this.beginPass(PASS_LABELS.attnPrefill);
    try {
      this.g4.attnPrefillRun(plan, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  attnPrefill(entries: PrefillEntry[], shape: StepShape, workspace: DeviceBuffer): void {
    this.attnPrefillRun(this.attnPrefillPrepare(entries, shape, workspace));
  }

  // One launch for every token of a chunk; q goes out as the f16 query of attnPrefill, and producer
  // layers store their K/V rows, bit-identical to the per-token reference kernels.
  attnPromptPrep(p: PromptPrep, shape: StepShape): void {
    const store = p.k !== undefined;
    if (store && (!p.v || !p.kWeight || !p.kCache || !p.vCache || p.maxSeqLen === undefined)) {
      throw new Error('attnPromptPrep: a producer layer needs k, v, kWeight, kCache, vCache and maxSeqLen');
    }
    const params = new Uniform([
      { u: shape.numQHeads }, { u: shape.numKvHeads }, { u: shape.headDim }, { u: p.nTokens }, { u: p.start },
      { f: p.eps === undefined ? 1e-6 : p.eps }, { f: p.theta }, { u: p.applyDivisor }, { u: store ? 1 : 0 },
      { u: p.maxSeqLen || 0 },
    ]);
    if (p.vtCache && !store) throw new Error('attnPromptPrep: vtCache on a layer that stores no rows');
    function ptr(b: DeviceBuffer | undefined): bigint | null { return b ? b.ptr : null; }
    const slot = this.beginPass(PASS_LABELS.attnPromptPrep);
    try {
      if (p.vtCache) {  // a producer layer: k, v, kWeight and the caches were checked above
        this.g4.attnPromptPrepVt(p.q.ptr, ptr(p.k) as bigint, ptr(p.v) as bigint, p.qWeight.ptr,
          ptr(p.kWeight) as bigint, ptr(p.ropeFreqs), ptr(p.ropeInvFreq), p.qOut.ptr, ptr(p.kCache) as bigint,
          ptr(p.vCache) as bigint, p.vtCache.ptr, params.bytes, this.stream);
      } else {
        this.g4.attnPromptPrep(p.q.ptr, ptr(p.k), ptr(p.v), p.qWeight.ptr, ptr(p.kWeight), ptr(p.ropeFreqs),
          ptr(p.ropeInvFreq), p.qOut.ptr, ptr(p.kCache), ptr(p.vCache), params.bytes, this.stream);
      }
    } finally {
      this.endPass(slot);
    }
  }

  // Several chunks' preps in one launch (chunks of several sequences in a batched prefill, or several layers
  // whose inputs are all ready); one head_dim for all, each chunk as attnPromptPrep would give it.
  attnPromptPrepMany(chunks: PromptPrep[], shape: StepShape): void {
    const REC = 128;  // g4_prompt_prep_entry: eleven pointers, then the ten 4-byte params fields
    const bytes = new Uint8Array(REC * chunks.length);
    const dv = new DataView(bytes.buffer);
    chunks.forEach(function (p, i) {
      const store = p.k !== undefined;
      if (store && (!p.v || !p.kWeight || !p.kCache || !p.vCache || p.maxSeqLen === undefined)) {
        throw new Error('attnPromptPrepMany: a producer layer needs k, v, kWeight, kCache, vCache and maxSeqLen');
      }
      if (p.vtCache && !store) throw new Error('attnPromptPrepMany: vtCache on a layer that stores no rows');
      const ptrs = [p.q, p.k, p.v, p.qWeight, p.kWeight, p.ropeFreqs, p.ropeInvFreq, p.qOut, p.kCache, p.vCache,
        p.vtCache];
      const o = i * REC;
      ptrs.forEach(function (b, j) { dv.setBigUint64(o + 8 * j, b ? b.ptr : BigInt(0), true); });
      const u = [shape.numQHeads, shape.numKvHeads, shape.headDim, p.nTokens, p.start];
      u.forEach(function (x, j) { dv.setUint32(o + 88 + 4 * j, x, true); });
      dv.setFloat32(o + 108, p.eps === undefined ? 1e-6 : p.eps, true);
      dv.setFloat32(o + 112, p.theta, true);
      dv.setUint32(o + 116, p.applyDivisor, true);
      dv.setUint32(o + 120, store ? 1 : 0, true);
      dv.setUint32(o + 124, p.maxSeqLen || 0, true);
    });
    const slot = this.beginPass(PASS_LABELS.attnPromptPrep);
    try {
      this.g4.attnPromptPrepMany(bytes, chunks.length, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  lmHeadWorkspaceSize(shape: LmHeadShape): number {
    return this.g4.lmHeadWorkspaceSize(shape.vocab, shape.hidden, shape.cap);
  }

  // lmHead -> logitSoftcap -> sample.argmax in one streaming pass: result[0] (u32) = the top-1 index;
  // logits (optional) = the softcapped logits, bit-identical to the three dispatches.
  lmHeadArgmax(hidden: DeviceBuffer, weight: DeviceBuffer, logits: DeviceBuffer | null, result: DeviceBuffer,
    workspace: DeviceBuffer, shape: LmHeadShape): void {
    if (weight.size < shape.vocab * shape.hidden * 2) throw new RangeError('lmHeadArgmax: weight too small');
    if (logits && logits.size < shape.vocab * 4) throw new RangeError('lmHeadArgmax: logits too small');
    const slot = this.beginPass(PASS_LABELS.lmHeadArgmax);
    try {
      this.g4.lmHeadArgmax(hidden.ptr, weight.ptr, logits ? logits.ptr : null, result.ptr, workspace.ptr,
        workspace.size, shape.vocab, shape.hidden, shape.cap, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  // attn.linearQKV (q, k, v in one launch: the three matrices read the same normed hidden state) and
  // attn.linearOut (src/engine.ts:2045-2051, 2096): each row bit-identical to a matmulQuant dispatch.
  // `label` names the pass for the profiler (default attn.linearQKV).
  linear(input: DeviceBuffer, n: number, segments: LinearSegment[], label?: string): void {
    if (input.size < n * 4) throw new RangeError('linear: input too small');
    const segs = segments.map(function (g, i) {
      if (g.weight.size < g.rows * n * 2) throw new RangeError('linear: segment ' + i + ' weight too small');
      if (g.out.size < g.rows * 4) throw new RangeError('linear: segment ' + i + ' out too small');
      return { weight: g.weight.ptr, out: g.out.ptr, rows: g.rows };
    });
    const slot = this.beginPass(label || PASS_LABELS.linear);
    try {
      this.g4.linear(input.ptr, n, segs, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  linearQkvPrepWorkspaceSize(shape: StepShape): number {
    return this.g4.linearQkvPrepWorkspaceSize(shape.numQHeads, shape.numKvHeads);
  }

  // attn.linearQKV with the producer-side prep as its epilogue (src/engine.ts:2045-2091 in one launch): q, k, v
  // projected, then normalised per head in place (q and k with RoPE at `position`) and, on producer layers (k
  // segments given), the k and v rows stored at row `slot` of the caches; every value bit-identical to the
  // reference's dispatches. The result feeds attnStep entries with qReady (and the row read from the cache).
  // format 'f16' (segments without meta), 'q8' or 'q4k'. workspace: linearQkvPrepWorkspaceSize bytes, cleared once.
  linearQkvPrep(input: DeviceBuffer, n: number, format: 'f16' | 'q8' | 'q4k', segments: QkvSegment[], p: QkvPrep,
    shape: StepShape, workspace: DeviceBuffer): void {
    if (input.size < n * 4) throw new RangeError('linearQkvPrep: input too small');
    const store = segments.length === 3;
    if (store && (!p.kWeight || !p.kCache || !p.vCache || p.maxSeqLen === undefined)) {
      throw new Error('linearQkvPrep: a producer layer needs kWeight, kCache, vCache and maxSeqLen');
    }
    const segs = segments.map(function (g) {
      return g.meta ? { weight: g.weight.ptr, meta: g.meta.ptr, out: g.out.ptr, rows: g.rows }
        : { weight: g.weight.ptr, out: g.out.ptr, rows: g.rows };
    });
    const params = new Uniform([
      { u: shape.numQHeads }, { u: shape.numKvHeads }, { u: shape.headDim }, { u: p.position }, { u: p.slot || 0 },
      { u: p.maxSeqLen || 0 }, { f: p.eps === undefined ? 1e-6 : p.eps }, { f: p.theta },
      { u: p.applyDivisor || 0 }, { u: store ? 1 : 0 },
    ]);
    function ptr(b: DeviceBuffer | undefined): bigint | null { return b ? b.ptr : null; }
    const slot = this.beginPass(PASS_LABELS.linearQkvPrep);
    try {
      this.g4.linearQkvPrep(input.ptr, n, format === 'q8' ? 1 : format === 'q4k' ? 2 : 0, segs, p.qWeight.ptr,
        ptr(p.kWeight), ptr(p.ropeFreqs), ptr(p.ropeInvFreq), ptr(p.kCache), ptr(p.vCache), params.bytes,
        workspace.ptr, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  // captureHidden for the attention block of one layer (src/engine.ts:2749-2815 with the stop points of
  // :2053-2095) on the fused kernels: runs the block for one token up to `stopAt` and returns the F32 contents
  // of the work buffer there. preRope*: attn.linearQKV alone (the raw projection). postRope*: linearQkvPrep,
  // whose epilogue leaves q and k post-norm, post-RoPE in place as fusedPerHeadNormRope leaves the engine's q
  // and k buffers (it also stores the producer's K/V row, which the engine does next in kvCacheStore).
  // attnOut: linearQkvPrep, then attnStep on the ready q with the row read from the cache. preRopeK,
  // preRopeV and postRopeK exist on KV-producer layers only, as in the engine.
  captureAttention(layer: AttnCaptureLayer, shape: StepShape, stopAt: AttnCapturePoint): Promise<Float32Array> {
    const producer = layer.segments.length === 3;
    if (!producer && (stopAt === 'preRopeK' || stopAt === 'preRopeV' || stopAt === 'postRopeK')) {
      return Promise.reject(new Error('captureAttention: ' + stopAt + ' exists on KV-producer layers only'));
    }
    const HD = shape.headDim;
    let src: DeviceBuffer;
    let count: number;
    try {
      if (stopAt === 'preRopeQ' || stopAt === 'preRopeK' || stopAt === 'preRopeV') {
        this.linear(layer.input, layer.n, layer.segments.map(function (g) {
          return { weight: g.weight, out: g.out, rows: g.rows };
        }));
        const i = stopAt === 'preRopeQ' ? 0 : stopAt === 'preRopeK' ? 1 : 2;
        src = layer.segments[i].out;
        count = (i === 0 ? shape.numQHeads : shape.numKvHeads) * HD;
      } else {
        this.linearQkvPrep(layer.input, layer.n, 'f16', layer.segments, layer.prep, shape, layer.prepWorkspace);
        if (stopAt === 'attnOut') {
          this.attnStep([{
            q: layer.segments[0].out, qWeight: layer.prep.qWeight, ropeFreqs: layer.prep.ropeFreqs,
            kCache: layer.kCache, vCache: layer.vCache, out: layer.out, seqLen: layer.seqLen,
            position: layer.prep.position, slidingWindow: layer.slidingWindow || 0, storeKv: false,
            theta: layer.prep.theta, applyDivisor: layer.prep.applyDivisor || 0, scale: layer.scale,
            eps: layer.prep.eps, qReady: true,
          }], shape, layer.stepWorkspace);
          src = layer.out;
          count = shape.numQHeads * HD;
        } else {
          src = layer.segments[stopAt === 'postRopeQ' ? 0 : 1].out;
          count = (stopAt === 'postRopeQ' ? shape.numQHeads : shape.numKvHeads) * HD;
        }
      }
    } catch (e) {
      return Promise.reject(e);
    }
    const out = new Float32Array(count);
    return this.readBufferAsync(src, 0, out).then(function () { return out; });
  }

  // The same with the engine's quantized weights: each row bit-identical to a matmulQ8 / matmulQ4K dispatch.
  linearQuant(input: DeviceBuffer, n: number, format: 'q8' | 'q4k', segments: QuantSegment[], label?: string): void {
    if (input.size < n * 4) throw new RangeError('linearQuant: input too small');
    const q8 = format === 'q8';
    const segs = segments.map(function (g, i) {
      if (g.weight.size < g.rows * (q8 ? n : n / 2)) throw new RangeError('linearQuant: segment ' + i + ' weight too small');
      if (g.meta.size < g.rows * (q8 ? n / 16 : n / 8)) throw new RangeError('linearQuant: segment ' + i + ' meta too small');
      if (g.out.size < g.rows * 4) throw new RangeError('linearQuant: segment ' + i + ' out too small');
      return { weight: g.weight.ptr, meta: g.meta.ptr, out: g.out.ptr, rows: g.rows };
    });
    const slot = this.beginPass(label || PASS_LABELS.linear);
    try {
      this.g4.linearQuant(input.ptr, n, q8 ? 1 : 2, segs, this.stream);
    } finally {
      this.endPass(slot);
    }
  }

  // ---- profiling: the engine's API and report (src/engine.ts:3085-3288, src/types.ts:490-515) ----

  getProfileCapability(): ProfileCapability {
    return { timestampQuerySupported: true, timestampQueryOnAdapterButUnrequested: false,
      querySlots: PROFILE_QUERY_SLOTS };
  }

  // Every pass enqueued from now on is timed, until disableProfile().
  enableProfile(): void {
    this.timer.on = true;
  }

  disableProfile(): void {
    this.timer.on = false;
  }

  resetProfileSamples(): void {
    this.timer.clear();
  }

  // Per label: percentiles over the samples of every forward collected so far, largest p50 first.
  getProfileReport(): ProfileReport {
    return this.timer.report();
  }

  // Ends a forward: waits (off the JS thread) for the timestamps of the passes enqueued since the last
  // collect, adds each pass's duration to its label's samples and their sum to the forward totals.
  collectProfileSamples(): Promise<void> {
    return this.timer.harvest();
  }

  // Opens a pass: the library kernels launched until endPass carry its two slots on their own dispatches
  // (the first one's start, the last one's end). Returns the pass's first slot, or -1 when it is untimed.
  private beginPass(label: string): number {
    return this.timer.begin(label);
  }

  private endPass(slot: number): void {
    if (slot >= 0) this.g4.queryEndPass();
  }

  synchronize(): void {
    this.g4.streamSynchronize(this.stream);
  }

  dispose(): void {
    if (!this.alive) return;
    this.g4.streamSynchronize(this.stream);
    this.timer.destroy();
    this.g4.streamDestroy(this.stream);
    this.alive = false;
  }
}

// The backend, selected once at init.
export function createAttention(device?: number, addonPath?: string): HipAttention {
  return new HipAttention(loadAddon(addonPath), device || 0);
}
