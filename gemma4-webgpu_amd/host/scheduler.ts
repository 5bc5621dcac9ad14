// Continuous-batching decode over the one-launch attention step.
//
// The engine decodes a single sequence (src/engine.ts:116, one kvPosition), so serving several
// sequences at once is host machinery of its own: requests wait in a FIFO queue, are admitted into a
// fixed number of cache slots, and leave when they finish, freeing their slot for the next request.
// Each layer of a token step is one attnStep launch over every active sequence: a ragged batch, one
// entry per sequence with its own length (the batched-decode workload of 64 sequences of 1K..32K
// rows is one such launch). beginToken() prepares every layer of the token step at once (one table
// upload per head_dim group, attnStepPrepareLayers), or, while the active sequences are the ones its
// plans were prepared for, advances those plans one token on the host (attnStepAdvance; prepared again
// every REPLAN_TOKENS tokens); stepLayer() then runs the layer's plan, or, without it, prepares that
// layer alone.
//
// Memory is taken once, at construction: one pool holds every slot's K and V cache rows of every
// KV-producer layer (consumer layers read their producer's rows, src/engine.ts:1518-1522), one holds
// the slots' q/k/v projections and attnOut, and one is the step's workspace, sized for a full batch.
// Nothing is allocated per token.

import type { DeviceBuffer, StepEntry, StepShape } from './attention';
import { HipAttention } from './attention';

// One layer of the model as the attention step sees it.
export interface LayerSpec {
  slidingWindow: number;      // 0 = global
  theta: number;
  applyDivisor?: number;      // 1 on global layers: rope_freqs divides the inverse frequencies
  kvSource: number;           // the layer whose cache this layer reads (its own index on producer layers)
  headDim?: number;           // default: the scheduler's headDim (E2B: 512 on global layers)
  qWeight: DeviceBuffer;      // attn_q_norm f16 [headDim]
  kWeight: DeviceBuffer;      // attn_k_norm f16 [headDim] (read on producer layers)
  ropeFreqs?: DeviceBuffer;   // f16 divisor table (applyDivisor layers)
  ropeInvFreq?: Float32Array; // host table from ropeInvFreqHost(): RoPE factors evaluated in prepare
  scale?: number;
  eps?: number;
}

export interface SchedulerConfig {
  shape: StepShape;           // numQHeads, numKvHeads, default headDim
  layers: LayerSpec[];
  maxBatch: number;           // cache slots: sequences decoded together
  maxSeqLen: number;          // cache rows per slot and producer layer
}

// beginToken prepares the plans again after this many tokens of advancing them (the part holding a full
// layer's last row takes the new rows meanwhile).
export const REPLAN_TOKENS = 32;

interface Waiting {
  id: string;
  length: number;
}

interface Active {
  slot: number;
  length: number;             // rows already in the cache; the next token sits at this position
}

// The slot bookkeeping alone (no device memory): FIFO admission into the lowest free slot, release,
// and the per-token advance.
export class SlotTable {
  readonly capacity: number;
  readonly maxSeqLen: number;
  private freeSlots: number[];
  private waiting: Waiting[];
  private active: Map<string, Active>;

  constructor(capacity: number, maxSeqLen: number) {
    if (!(capacity >= 1) || Math.floor(capacity) !== capacity) throw new RangeError('SlotTable: capacity must be a positive integer');
    if (!(maxSeqLen >= 1) || Math.floor(maxSeqLen) !== maxSeqLen) throw new RangeError('SlotTable: maxSeqLen must be a positive integer');
    this.capacity = capacity;
    this.maxSeqLen = maxSeqLen;
    this.freeSlots = [];
    for (let s = 0; s < capacity; s++) this.freeSlots.push(s);
    this.waiting = [];
    this.active = new Map();
  }

  // A request joins the queue; `length` = rows its caches will hold when admitted (its prompt, filled
  // by prefill), so its first decoded token sits at position `length`.
  submit(id: string, length: number): void {
    if (this.active.has(id) || this.waiting.some(function (w) { return w.id === id; })) {
      throw new Error(`submit: sequence ${id} is already queued or active`);
    }
    if (!(length >= 0) || Math.floor(length) !== length || length >= this.maxSeqLen) {
      throw new RangeError(`submit: sequence ${id}: length ${length} outside [0, ${this.maxSeqLen - 1}]`);
    }
    this.waiting.push({ id: id, length: length });
  }

  // Moves waiting requests into free slots, oldest first; returns the admitted ids.
  admit(): string[] {
    const done: string[] = [];
    while (this.waiting.length && this.freeSlots.length) {
      const w = this.waiting.shift() as Waiting;
      const slot = this.freeSlots.shift() as number;
      this.active.set(w.id, { slot: slot, length: w.length });
      done.push(w.id);
    }
    return done;
  }

  // A finished (or cancelled) sequence leaves: its slot is free for the next admission.
  release(id: string): void {
    const a = this.active.get(id);
    if (a) {
      this.active.delete(id);
      this.freeSlots.push(a.slot);
      this.freeSlots.sort(function (x, y) { return x - y; });
      return;
    }
    const i = this.waiting.findIndex(function (w) { return w.id === id; });
    if (i < 0) throw new Error(`release: unknown sequence ${id}`);
    this.waiting.splice(i, 1);
  }

  // Active sequences in admission order (the order of a step's entries).
  activeIds(): string[] {
    return Array.from(this.active.keys());
  }

  waitingIds(): string[] {
    return this.waiting.map(function (w) { return w.id; });
  }

  isActive(id: string): boolean {
    return this.active.has(id);
  }

  slotOf(id: string): number {
    return this.get(id).slot;
  }

  lengthOf(id: string): number {
    return this.get(id).length;
  }

  // True when the sequence's caches are full: it cannot take another token.
  isFull(id: string): boolean {
    return this.get(id).length >= this.maxSeqLen;
  }

  // After every layer of a token step: each active sequence holds one more row.
  advance(): void {
    const self = this;
    this.active.forEach(function (a, id) {
      if (a.length >= self.maxSeqLen) throw new RangeError(`advance: sequence ${id} is full`);
    });
    this.active.forEach(function (a) { a.length += 1; });
  }

  private get(id: string): Active {
    const a = this.active.get(id);
    if (!a) throw new Error(`sequence ${id} is not active`);
    return a;
  }
}

function view(b: DeviceBuffer, offset: number, size: number): DeviceBuffer {
  if (offset + size > b.size) throw new RangeError(`view: ${offset}+${size} > ${b.size}`);
  return { ptr: b.ptr + BigInt(offset), size: size };
}

export class DecodeScheduler {
  readonly table: SlotTable;
  private readonly att: HipAttention;
  private readonly cfg: SchedulerConfig;
  private readonly producers: number[];        // producer layer indices, in order
  private readonly cacheOffset: number[];      // per producer: byte offset of slot 0's K rows in the pool
  private readonly slotCacheBytes: number;     // bytes of one slot's caches over all producers
  private readonly maxHd: number;
  private pool: DeviceBuffer;
  private work: DeviceBuffer;
  private workspace: DeviceBuffer;
  private readonly groups: { layers: number[]; workspace: DeviceBuffer }[];  // layers per head_dim, in order
  private tokenPlans: Uint8Array[] | null;     // beginToken's plans, one per layer
  private tokenIds: string;                    // the active sequences they were prepared for
  private token: number;                       // tokens stepped (advance() calls)
  private plansToken: number;                  // the token the plans are at
  private sincePrepare: number;                // tokens the plans were advanced since their prepare
  prepares: number;                            // beginToken calls that prepared (the rest advanced)
  private alive: boolean;

  constructor(att: HipAttention, cfg: SchedulerConfig) {
    const nl = cfg.layers.length;
    if (!nl) throw new RangeError('DecodeScheduler: no layers');
    this.att = att;
    this.cfg = cfg;
    this.table = new SlotTable(cfg.maxBatch, cfg.maxSeqLen);
    const nkh = cfg.shape.numKvHeads;
    this.producers = [];
    this.cacheOffset = [];
    let maxHd = 0;
    let off = 0;
    for (let l = 0; l < nl; l++) {
      const L = cfg.layers[l];
      const hd = this.hdOf(l);
      if (hd % 256 !== 0 || hd > 512) throw new RangeError(`layer ${l}: head_dim ${hd} unsupported (256 or 512)`);
      maxHd = Math.max(maxHd, hd);
      const src = L.kvSource;
      if (!(src >= 0 && src <= l) || cfg.layers[src].kvSource !== src) {
        throw new RangeError(`layer ${l}: kvSource ${src} is not an earlier (or the same) producer layer`);
      }
      if (this.hdOf(src) !== hd) throw new RangeError(`layer ${l}: head_dim differs from its producer's`);
      if (src === l) {
        this.producers.push(l);
        this.cacheOffset[l] = off;
        off += 2 * cfg.maxSeqLen * nkh * hd * 2;  // K then V rows of one slot
      }
    }
    this.maxHd = maxHd;
    this.slotCacheBytes = off;
    this.pool = att.createBuffer(cfg.maxBatch * off);
    // Per slot: q [NQH][HD], k and v [NKH][HD], out [NQH][HD], f32, at the largest head_dim.
    this.work = att.createBuffer(cfg.maxBatch * this.slotWorkBytes());
    let ws = 0;
    for (let l = 0; l < nl; l++) ws = Math.max(ws, att.attnStepWorkspaceSize(cfg.maxBatch, this.shapeOf(l)));
    this.workspace = att.createBuffer(ws);
    // beginToken: a layers workspace per head_dim group, for a full batch
    const byHd: number[][] = [];
    for (let l = 0; l < nl; l++) {
      let list: number[] | null = null;
      for (const x of byHd) if (this.hdOf(x[0]) === this.hdOf(l)) list = x;
      if (list) list.push(l);
      else byHd.push([l]);
    }
    this.groups = [];
    for (const layers of byHd) {
      const bytes = att.attnStepLayersWorkspaceSize(layers.length, this.shapeOf(layers[0]), cfg.maxBatch);
      this.groups.push({ layers: layers, workspace: att.createBuffer(bytes) });
    }
    this.tokenPlans = null;
    this.tokenIds = '';
    this.token = 0;
    this.plansToken = -1;
    this.sincePrepare = 0;
    this.prepares = 0;
    this.alive = true;
  }

  submit(id: string, length: number): void { this.table.submit(id, length); }
  admit(): string[] {
    const admitted = this.table.admit();
    if (admitted.length) this.tokenPlans = null;  // the active set changed: prepare at the next beginToken
    return admitted;
  }
  release(id: string): void {
    this.tokenPlans = null;
    this.table.release(id);
  }
  activeIds(): string[] { return this.table.activeIds(); }

  // The sequence's K / V cache of `layer` (its producer's rows on consumer layers): f16 [maxSeqLen][NKH][HD].
  kCache(id: string, layer: number): DeviceBuffer { return this.cacheView(id, layer, 0); }
  vCache(id: string, layer: number): DeviceBuffer { return this.cacheView(id, layer, 1); }

  // The sequence's projections for the current layer (written by attn.linearQKV; k and v on producer
  // layers only) and its attnOut (read by attn.linearOut), f32, sized for the layer's head_dim.
  q(id: string, layer: number): DeviceBuffer { return this.workView(id, 0, this.cfg.shape.numQHeads * this.hdOf(layer)); }
  k(id: string, layer: number): DeviceBuffer { return this.workView(id, 1, this.cfg.shape.numKvHeads * this.hdOf(layer)); }
  v(id: string, layer: number): DeviceBuffer { return this.workView(id, 2, this.cfg.shape.numKvHeads * this.hdOf(layer)); }
  out(id: string, layer: number): DeviceBuffer { return this.workView(id, 3, this.cfg.shape.numQHeads * this.hdOf(layer)); }

  // The entries of one layer's step: every active sequence at its next position.
  entries(layer: number): StepEntry[] {
    const L = this.cfg.layers[layer];
    if (!L) throw new RangeError(`entries: no layer ${layer}`);
    const self = this;
    return this.table.activeIds().map(function (id) {
      const length = self.table.lengthOf(id);
      if (length >= self.cfg.maxSeqLen) throw new RangeError(`step: sequence ${id} is full (${length} rows)`);
      const producer = L.kvSource === layer;
      const e: StepEntry = {
        q: self.q(id, layer), qWeight: L.qWeight,
        kCache: self.kCache(id, layer), vCache: self.vCache(id, layer), out: self.out(id, layer),
        seqLen: length + 1, position: length, slidingWindow: L.slidingWindow, storeKv: producer,
        theta: L.theta, applyDivisor: L.applyDivisor || 0, scale: L.scale, eps: L.eps,
      };
      if (producer) {  // consumers project only q: their producer stored this token's row already
        e.k = self.k(id, layer);
        e.v = self.v(id, layer);
        e.kWeight = L.kWeight;
      }
      if (L.ropeFreqs) e.ropeFreqs = L.ropeFreqs;
      if (L.ropeInvFreq) e.ropeInvFreq = L.ropeInvFreq;
      return e;
    });
  }

  // Every layer of the token step made ready at once, for the active sequences (the engine patches every
  // layer's uniforms once per token, src/engine.ts:1967-1987): when the previous token's plans were made
  // for the same sequences, each advances one token on the host (attnStepAdvance, nothing enqueued);
  // otherwise, and every REPLAN_TOKENS tokens, one attnStepPrepareLayers per head_dim group, one table
  // upload each. Call after admit/release, before the token's first layer; stepLayer then runs the
  // plans. Returns the number of sequences.
  beginToken(): number {
    const ids = this.table.activeIds();
    const key = ids.join('\n');
    if (this.tokenPlans && this.tokenIds === key) {
      if (this.plansToken === this.token) return ids.length;
      if (this.plansToken + 1 === this.token && this.sincePrepare + 1 < REPLAN_TOKENS) {
        for (const p of this.tokenPlans) this.att.attnStepAdvance(p, 1);
        this.sincePrepare++;
        this.plansToken = this.token;
        return ids.length;
      }
    }
    this.tokenPlans = null;
    if (!ids.length) return 0;
    const plans: Uint8Array[] = new Array(this.cfg.layers.length);
    for (const g of this.groups) {
      const ents: StepEntry[] = [];
      for (const l of g.layers) for (const e of this.entries(l)) ents.push(e);
      const ps = this.att.attnStepPrepareLayers(ents, this.shapeOf(g.layers[0]), g.workspace, ids.length);
      g.layers.forEach(function (l, i) { plans[l] = ps[i]; });
    }
    this.tokenPlans = plans;
    this.tokenIds = key;
    this.plansToken = this.token;
    this.sincePrepare = 0;
    this.prepares++;
    return ids.length;
  }

  // One layer of the token step for every active sequence: one attention launch (plus the split
  // merge), from beginToken's plan when it was prepared for these sequences, else prepared here.
  // Returns the number of sequences stepped.
  stepLayer(layer: number): number {
    const ids = this.table.activeIds();
    if (this.tokenPlans && this.plansToken === this.token && this.tokenIds === ids.join('\n')) {
      this.att.attnStepRun(this.tokenPlans[layer]);
      return ids.length;
    }
    const ents = this.entries(layer);
    if (ents.length) this.att.attnStep(ents, this.shapeOf(layer), this.workspace);
    return ents.length;
  }

  // After the last layer of a token: every active sequence holds one more row (the plans are now one
  // token behind; the next beginToken advances them).
  advance(): void {
    this.token++;
    this.table.advance();
  }

  dispose(): void {
    if (!this.alive) return;
    this.att.synchronize();
    this.att.destroyBuffer(this.pool);
    this.att.destroyBuffer(this.work);
    this.att.destroyBuffer(this.workspace);
    for (const g of this.groups) this.att.destroyBuffer(g.workspace);
    this.alive = false;
  }

  private hdOf(layer: number): number {
    return this.cfg.layers[layer].headDim || this.cfg.shape.headDim;
  }

  private shapeOf(layer: number): StepShape {
    return { numQHeads: this.cfg.shape.numQHeads, numKvHeads: this.cfg.shape.numKvHeads, headDim: this.hdOf(layer) };
  }

  private slotWorkBytes(): number {
    const s = this.cfg.shape;
    return (2 * s.numQHeads + 2 * s.numKvHeads) * this.maxHd * 4;
  }

  private cacheView(id: string, layer: number, which: number): DeviceBuffer {
    const L = this.cfg.layers[layer];
    if (!L) throw new RangeError(`no layer ${layer}`);
    const src = L.kvSource;
    const rows = this.cfg.maxSeqLen * this.cfg.shape.numKvHeads * this.hdOf(src) * 2;
    const off = this.table.slotOf(id) * this.slotCacheBytes + this.cacheOffset[src] + which * rows;
    return view(this.pool, off, rows);
  }

  // Work rows of a slot: q, k, v, out at fixed offsets for the largest head_dim (16-byte aligned).
  private workView(id: string, which: number, floats: number): DeviceBuffer {
    const s = this.cfg.shape;
    const hd = this.maxHd;
    const starts = [0, s.numQHeads * hd, (s.numQHeads + s.numKvHeads) * hd, (s.numQHeads + 2 * s.numKvHeads) * hd];
    const off = this.table.slotOf(id) * this.slotWorkBytes() + starts[which] * 4;
    return view(this.work, off, floats * 4);
  }
}
