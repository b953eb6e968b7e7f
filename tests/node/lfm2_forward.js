'use strict'
/*
 * A whole LFM2-shaped forward through HipGpu alone, as the reference's
 * Engine.forwardBatch drives its backend (src/engine.ts:8875-9303): the
 * weights uploaded as GGUF Q4_0 blocks and repacked by the addon, a prompt
 * through the prefill GEMMs, greedy decode steps through the few-token
 * GEMVs with their epilogues, then one verify batch of a token and 4
 * drafts whose accept and conv-state rollback run on the device
 * (src/handler.ts:1811-1887, Engine.accept src/engine.ts:8063-8086), and
 * two more steps after the rollback. Usage:
 *   node lfm2_forward.js <folder>
 * The folder holds model.json (the shape, tensor files, prompt, drafts);
 * the script writes the picks to out.json and each step's logits to
 * logits_<step>.bin for the Python side to compare with the oracle.
 */
const assert = require('assert')
const fs = require('fs')
const path = require('path')

const hip = require(path.join(__dirname, '..', '..', 'webgllm_amd', 'node', 'index.js'))

const { GL } = hip
const C = hip.constants
const MAX_ROWS = 8
const PRESCALE = 32 // the reference's PRESCALE (src/gpu/kernels.ts:89)

/** Stored row p of a gate|up matrix holds logical row order[p]: (gate 2i, gate 2i+1, up 2i, up 2i+1). */
function gateUpRowOrder (F) {
  const order = new Int32Array(2 * F)
  for (let i = 0; i < F / 2; i++) order.set([2 * i, 2 * i + 1, F + 2 * i, F + 2 * i + 1], 4 * i)
  return order
}

/** Engine.ropeTable (src/engine.ts:1292-1312): cos | sin in doubles, stored as floats. */
function ropeTable (theta, hd, ctx) {
  const half = hd / 2
  const rows = 1024 + Math.ceil(ctx / 1024)
  const t = new Float32Array(rows * hd)
  for (let r = 0; r < rows; r++) {
    const pos = r < 1024 ? r : (r - 1024) * 1024
    for (let i = 0; i < half; i++) {
      const ang = pos * Math.pow(theta, (-2 * i) / hd)
      t[r * hd + i] = Math.cos(ang)
      t[r * hd + half + i] = Math.sin(ang)
    }
  }
  return { table: t, rows }
}

class Lfm2 {
  constructor (gpu, dir, cfg) {
    this.gpu = gpu
    this.ops = gpu.ops
    this.cfg = cfg
    const D = cfg.hidden
    const F = cfg.intermediate
    const W = cfg.convKernel
    const hd = cfg.headDim
    const ctx = cfg.ctx
    this.shape = { heads: cfg.heads, kvHeads: cfg.kvHeads, headDim: hd, rotatedDims: hd, eps: cfg.eps, useNorm: 1 }
    const read = (name) => fs.readFileSync(path.join(dir, cfg.tensors[name]))
    const floats = (name, n) => {
      const b = read(name)
      assert.strictEqual(b.length, n * 4, name)
      return gpu.texture(GL.R32F, n, 1, { pixels: b })
    }
    // a Q4_0 matrix: the file's blocks on the device, repacked there (srcRows: the stored row order)
    const q4 = (name, N, K, order) => {
      const src = read(name)
      assert.strictEqual(src.length, N * (K / 32) * 18, name)
      const tsrc = gpu.texture(GL.R8UI, src.length, 1, { pixels: src })
      const sizes = hip.quantSizes(N, K)
      const w = {
        N, K, layout: C.LAYOUT_ROWGROUP, zero: C.ZERO_8,
        quants: gpu.texture(GL.R8UI, sizes.quants, 1),
        scales: gpu.texture(GL.R8UI, sizes.scales, 1)
      }
      this.ops.repack('q4_0', w, 0, N, tsrc, order || null)
      gpu.delete(tsrc)
      return w
    }
    this.embedding = q4('embedding', cfg.vocab, D)
    this.finalNorm = floats('final_norm', D)
    this.layers = cfg.layerTypes.map((type, i) => {
      const p = `layers.${i}.`
      const l = {
        type,
        opNorm: floats(p + 'op_norm', D),
        ffnNorm: floats(p + 'ffn_norm', D),
        gateUp: q4(p + 'gate_up', 2 * F, D, gateUpRowOrder(F)),
        down: q4(p + 'down', D, F)
      }
      if (type === 'conv') {
        l.inProj = q4(p + 'in_proj', 3 * D, D)
        l.outProj = q4(p + 'out_proj', D, D)
        l.taps = floats(p + 'taps', D * W)
        l.state = gpu.texture(GL.R32F, D, W - 1)
        l.prefixes = gpu.texture(GL.R32F, D * (W - 1), MAX_ROWS)
        gpu.zero(l.state)
      } else {
        const qkvRows = (cfg.heads + 2 * cfg.kvHeads) * hd
        l.qkv = q4(p + 'qkv', qkvRows, D)
        l.o = q4(p + 'o', D, cfg.heads * hd)
        l.qNorm = floats(p + 'q_norm', hd)
        l.kNorm = floats(p + 'k_norm', hd)
        const kvd = cfg.kvHeads * hd
        l.kCache = gpu.texture(GL.R8UI, ctx * kvd * 2, 1)
        l.vCache = gpu.texture(GL.R8UI, ctx * kvd * 2, 1)
        gpu.zero(l.kCache)
        gpu.zero(l.vCache)
      }
      return l
    })
    const rope = ropeTable(cfg.ropeTheta, hd, ctx)
    this.rope = gpu.texture(GL.R32F, hd, rope.rows, { pixels: rope.table })
    this.ropeRows = rope.rows
    // the batch's activations (Engine's few-token buffers)
    const R = MAX_ROWS
    const A = cfg.heads * hd
    const f32 = (n, rows) => gpu.texture(GL.R32F, n, rows)
    const f16 = (n, rows) => gpu.texture(GL.R8UI, n * 2, rows)
    const i32 = (n) => gpu.texture(GL.R32I || GL.R32UI, n, 1)
    this.ids = i32(R)
    this.pos = i32(1)
    this.h = f32(D, R)
    this.x16 = f16(D, R)
    this.c16 = f16(D, R)
    this.parts = f32(D / 4, R)
    this.qkvOut = f32((cfg.heads + 2 * cfg.kvHeads) * hd, R)
    this.q = f32(A, R)
    this.att16 = f16(A, R)
    this.ff16 = f16(F, R)
    this.bcx = f32(3 * D, R)
    this.logits = f32(cfg.vocab, R)
    this.nextIds = i32(R)
    this.tops = f32(R, 1)
    this.argmaxScratch = gpu.texture(GL.R8UI, this.ops.argmaxScratchBytes(R, cfg.vocab), 1)
    // attention scratch: its counters start at zero and every call leaves them so
    this.attnScratch = gpu.texture(GL.R8UI, this.ops.attnScratchBytes(R, cfg.heads, hd, ctx), 1)
    gpu.zero(this.attnScratch)
    // the prompt batch's buffers (the prefill GEMMs' rows)
    const P = cfg.maxPrompt
    this.pre = {
      ids: i32(P), h: f32(D, P), rs: f32(P, 1), x16: f16(D, P), c16: f16(D, P), bcx: f32(3 * D, P),
      qkv: f32((cfg.heads + 2 * cfg.kvHeads) * hd, P), q: f32(A, P), att16: f16(A, P), ff16: f16(F, P)
    }
    // verify on the device: the conv layers' rollback table, the history, the kept log
    const convs = this.layers.filter((l) => l.type === 'conv')
    this.convTable = this.ops.convStates(convs.map((l) => ({ prefixes: l.prefixes, state: l.state, dim: D, width: W })), MAX_ROWS)
    this.nConv = convs.length
    this.hist = i32(ctx + 1)
    this.keptLog = i32(16)
    this.cursor = i32(1)
    gpu.zero(this.hist)
    gpu.zero(this.cursor)
    this.position = 0
  }

  setRows (tex, values) { this.gpu.writeBytes(tex, 0, Int32Array.from(values)) }

  /** The input side of a GEMV that reads the prescaled residual (the normed matmul, kernels.ts:744-895). */
  normIn (ep) {
    const D = this.cfg.hidden
    return Object.assign(ep, { normParts: this.parts, nParts: D / 4, ldPartsIn: D / 4, normCount: D, eps: this.cfg.eps, normMult: PRESCALE })
  }

  /** h += result; the next norm's prescaled input and its sums of squares (addScaled + rmsOfAdd). */
  residualOut (nextNorm) {
    const D = this.cfg.hidden
    return { mode: C.EPI_STORE, residual: this.h, ldResidual: D, out16: this.x16, ldOut16: D, out16W: nextNorm, normMultOut: PRESCALE, partsOut: this.parts, ldPartsOut: D / 4 }
  }

  nextNorm (i) { return i + 1 < this.layers.length ? this.layers[i + 1].opNorm : this.finalNorm }

  /** One batch of M <= 8 rows (ids at positions pos ..): the greedy picks into nextIds. */
  forwardRows (M, keepPrefixes) {
    const { ops, cfg } = this
    const D = cfg.hidden
    const F = cfg.intermediate
    ops.embed(this.embedding, this.ids, M, this.h, {
      mode: C.EPI_STORE, out16: this.x16, ldOut16: D, out16W: this.layers[0].opNorm, normMultOut: PRESCALE, partsOut: this.parts, ldPartsOut: D / 4
    })
    this.layers.forEach((l, i) => {
      if (l.type === 'conv') {
        ops.gemv(l.inProj, this.x16, M, this.bcx, this.normIn({ mode: C.EPI_STORE }))
        ops.shortConv(this.bcx, M, D, cfg.convKernel, l.taps, l.state, l.state, keepPrefixes ? l.prefixes : null, this.c16)
        ops.gemv(l.outProj, this.c16, M, this.h, this.residualOut(l.ffnNorm))
      } else {
        ops.gemv(l.qkv, this.x16, M, this.qkvOut, this.normIn({ mode: C.EPI_STORE }))
        ops.headPrep(this.qkvOut, M, this.shape, l.qNorm, l.kNorm, this.rope, this.ropeRows, this.pos, this.q, l.kCache, l.vCache, cfg.ctx)
        ops.attnDecode(this.q, M, this.shape, l.kCache, l.vCache, this.pos, cfg.ctx, this.att16, this.attnScratch)
        ops.gemv(l.o, this.att16, M, this.h, this.residualOut(l.ffnNorm))
      }
      ops.gemv(l.gateUp, this.x16, M, null, this.normIn({ mode: C.EPI_SWIGLU, out16: this.ff16, ldOut16: F }))
      ops.gemv(l.down, this.ff16, M, this.h, this.residualOut(this.nextNorm(i)))
    })
    ops.gemv(this.embedding, this.x16, M, this.logits, this.normIn({ mode: C.EPI_STORE }))
    ops.argmax(this.logits, M, cfg.vocab, this.nextIds, this.argmaxScratch, this.tops)
  }

  /** A prompt batch through the prefill GEMMs (Engine.matmul, src/engine.ts:4969-5234), then the head of its last T rows. */
  prefill (tokens) {
    const { ops, cfg, gpu, pre } = this
    const D = cfg.hidden
    const M = tokens.length
    const eps = cfg.eps
    this.setRows(pre.ids, tokens)
    this.setRows(this.pos, [this.position])
    ops.embed(this.embedding, pre.ids, M, pre.h)
    this.layers.forEach((l) => {
      ops.normToH2(pre.h, M, D, l.opNorm, eps, pre.x16, pre.rs)
      if (l.type === 'conv') {
        ops.gemm(l.inProj, pre.x16, M, pre.bcx, { rowScale: pre.rs })
        ops.shortConv(pre.bcx, M, D, cfg.convKernel, l.taps, l.state, l.state, null, pre.c16)
        ops.gemm(l.outProj, pre.c16, M, pre.h, { residual: pre.h })
      } else {
        ops.gemm(l.qkv, pre.x16, M, pre.qkv, { rowScale: pre.rs })
        ops.headPrep(pre.qkv, M, this.shape, l.qNorm, l.kNorm, this.rope, this.ropeRows, this.pos, pre.q, l.kCache, l.vCache, cfg.ctx)
        ops.attnPrefill(pre.q, M, this.shape, l.kCache, l.vCache, this.pos, cfg.ctx, pre.att16)
        ops.gemm(l.o, pre.att16, M, pre.h, { residual: pre.h })
      }
      ops.normToH2(pre.h, M, D, l.ffnNorm, eps, pre.x16, pre.rs)
      ops.gemmSwiglu(l.gateUp, pre.x16, M, pre.ff16, pre.rs)
      ops.gemm(l.down, pre.ff16, M, pre.h, { residual: pre.h })
    })
    // the picks of the last batch of 8 (the engine returns those)
    const T = M % MAX_ROWS || MAX_ROWS
    const r0 = M - T
    const x16 = gpu.view(pre.x16, r0 * D * 2)
    const rs = gpu.view(pre.rs, r0 * 4)
    ops.normToH2(gpu.view(pre.h, r0 * D * 4), T, D, this.finalNorm, eps, x16, rs)
    ops.gemv(this.embedding, x16, T, this.logits, { mode: C.EPI_STORE, rowScale: rs })
    ops.argmax(this.logits, T, cfg.vocab, this.nextIds, this.argmaxScratch, this.tops)
    this.position += M
    return T
  }

  picks (M) { return Array.from(new Int32Array(this.gpu.readBytes(this.nextIds, 0, M * 4))) }
  logitsOf (M) { return Buffer.from(this.gpu.readBytes(this.logits, 0, M * this.cfg.vocab * 4)) }
}

async function main () {
  const dir = process.argv[2]
  const cfg = JSON.parse(fs.readFileSync(path.join(dir, 'model.json')))
  const gpu = new hip.HipGpu(0)
  const model = new Lfm2(gpu, dir, cfg)
  const out = { steps: [] }
  const save = (name, M, picks) => {
    fs.writeFileSync(path.join(dir, `logits_${name}.bin`), model.logitsOf(M))
    out.steps.push({ name, rows: M, picks })
  }
  // the prompt
  const T = model.prefill(cfg.prompt)
  const promptPicks = model.picks(T)
  save('prompt', T, promptPicks)
  // greedy decode, one row a step, eager launches behind a fence a step
  let token = promptPicks[T - 1]
  for (let s = 0; s < cfg.decodeSteps; s++) {
    model.setRows(model.ids, [token])
    model.setRows(model.pos, [model.position])
    model.forwardRows(1, false)
    const f = gpu.fence()
    await gpu.wait(f)
    const p = model.picks(1)
    save(`decode${s}`, 1, p)
    token = p[0]
    model.position += 1
  }
  // one verify batch: the last token and 4 drafts; accept and rollback on the device
  const rows = 1 + cfg.drafts.length
  model.setRows(model.ids, [token].concat(cfg.drafts))
  model.setRows(model.pos, [model.position])
  model.forwardRows(rows, true)
  const D = cfg.hidden
  model.ops.verifyAccept(model.nextIds, rows, model.convTable, model.nConv, (cfg.convKernel - 1) * D, model.pos, model.ids,
    model.hist, cfg.ctx + 1, model.keptLog, 16, model.cursor)
  const vp = model.picks(rows)
  save('verify', rows, vp)
  const pos = new Int32Array(gpu.readBytes(model.pos, 0, 4))[0]
  const kept = new Int32Array(gpu.readBytes(model.keptLog, 0, 4))[0]
  const hist = Array.from(new Int32Array(gpu.readBytes(model.hist, (model.position + 1) * 4, kept * 4)))
  const next = new Int32Array(gpu.readBytes(model.ids, 0, 4))[0]
  assert.strictEqual(pos, model.position + kept)
  assert.deepStrictEqual(hist, vp.slice(0, kept))
  assert.strictEqual(next, vp[kept - 1])
  out.verify = { kept, position: pos, written: hist }
  model.position = pos
  // decoding goes on from the rolled-back conv states and the kept cache rows
  token = next
  for (let s = 0; s < cfg.afterSteps; s++) {
    model.setRows(model.ids, [token])
    model.setRows(model.pos, [model.position])
    model.forwardRows(1, false)
    const p = model.picks(1)
    save(`after${s}`, 1, p)
    token = p[0]
    model.position += 1
  }
  // operands smaller than their shapes are refused before any launch
  let err = null
  try { model.ops.gemv(model.embedding, model.x16, 8, model.tops) } catch (e) { err = e }
  assert.ok(err instanceof hip.GpuError && err.code === 'WG_ERR_INVALID', String(err))
  out.bytes = gpu.bytes
  gpu.dispose()
  fs.writeFileSync(path.join(dir, 'out.json'), JSON.stringify(out))
  process.stdout.write(JSON.stringify({ ok: true, steps: out.steps.length }) + '\n')
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : e)
  process.exit(1)
})
