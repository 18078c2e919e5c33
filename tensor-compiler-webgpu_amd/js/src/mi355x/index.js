'use strict';
// The MI355X backend's entry points, as the reference's harnesses would import
// them in place of src/gpu/runtime.js, src/fusion/lower-fused.js,
// src/fusion/trainer-fused.js and src/fusion/bench.js of
// abho7/tensor-compiler-webgpu:
//   lowerMI355X(graph, { sabotage })            for lowerFused / lower
//   HipRunner.create(); runner.run(...)         for GpuRunner.create / run
//   runner.runLocal(graph, lowered, values)     for harness-m3b.js runLocal
//   fusedStep(step); new HipTrainer(...)        for fusedStep / FusedTrainer
//   fusedForward(fwd)                           for harness-m4.js's fuse + lowerFused of a forward pass
//   new HipBench(runner); bench.time(...)       for Bench.time; verdict, summarize
// and this backend's own additions: fuseAttention(fused, { keep }) (attention
// as one fused node, after the reference's fuse) and planArena (the liveness
// placement Program uses with { arena: { keep } }).
// Graphs are the reference's own (its Graph objects, or their toJSON form with
// fused nodes from its fuse()).

const { lowerMI355X, kernelSources } = require('./lower');
const { HipRunner, Program, precompile } = require('./runner');
const { fusedStep, fusedForward, HipTrainer } = require('./trainer');
const { HipBench, summarize, verdict } = require('./bench');
const { fuseAttention } = require('../fusion/attention');
const { planArena } = require('./arena');

module.exports = { lowerMI355X, kernelSources, HipRunner, Program, precompile, fusedStep, fusedForward, HipTrainer, HipBench, summarize, verdict,
  fuseAttention, planArena };
