! fgpt_drop_in.f90 -- the fortran_gpt model API, routed to the gfx950 engine.
!
! gpt_forward, gpt_step and gpt_step_multi keep the names and argument lists
! of the reference (src/lib/fortran_gpt.f90:54-92, src/lib/fortran_kv.f90:
! 26-55 and :160-189), so an app switches by changing its `use` line.
! load_gpt_weights keeps the reference loader's signature and .npy layout
! (src/lib/load_weights.f90:830-874) with its loud failures.
!
! What changes under the same arguments:
!  - The weights are uploaded to HBM (bf16, exact) on the first call and kept
!    there: one engine model per distinct (weight arrays, dims, eps), so a
!    caller that alternates the full depth and a truncated n_layer over the
!    same stacked arrays (spec_bench's drafter) keeps one upload of each.
!    Weights changed in place are not seen: call fgpt_release() after
!    changing them.
!  - The KV cache lives in HBM: one device cache per caller cache (the
!    address of cache_k) and model, B and maxT, so distinct host caches stay
!    distinct. cache_k / cache_v are accepted and left untouched; cache_len
!    is honoured in and out exactly as in the reference (resetting it to 0
!    starts a new sequence, rolling it back re-uses the rows below it); a
!    cache_len past the positions that cache has computed stops the program.
!  - RoPE rows are taken from the caller's tables on every call (the rows of
!    the positions being computed), as the reference uses them.
!  - Errors stop the program with the engine's message, the reference's
!    loud-failure convention (print + exit, or error stop).
!  - fgpt_forward_f16(.true.) lets gpt_forward passes of more than 128 rows
!    run as single-term fp16 MFMA work (FG_OPT_FORWARD_F16: logits within
!    ~4e-4 x max|logit| instead of ~5e-6, ~1.4x faster at 2048 tokens) for
!    callers whose forwards no decode follows (eval_bpb); gpt_step and
!    gpt_step_multi are unaffected. Off unless asked for.
module fgpt_drop_in_mod
  use, intrinsic :: iso_c_binding
  use, intrinsic :: iso_fortran_env, only: error_unit
  use fgpt_c
  implicit none
  private
  public :: gpt_forward, gpt_step, gpt_step_multi, load_gpt_weights, fgpt_release, &
      fgpt_handles, accept_prefix, lookup_draft, sample_next, fgpt_forward_f16

  ! engine models by (weight array addresses, dims, eps) and device caches
  ! by (address of the caller's cache_k, model, B, maxT)
  integer, parameter :: NMODELS = 4, NCACHES = 8
  type model_slot
    type(c_ptr) :: h = c_null_ptr
    integer(c_intptr_t) :: key(8) = 0
    integer :: dims(6) = -1
    real(c_float) :: eps = 0.0
  end type model_slot
  type kv_slot
    type(c_ptr) :: h = c_null_ptr
    integer(c_intptr_t) :: cache = 0
    integer :: model = 0, bb = -1, maxt = -1
  end type kv_slot
  type(model_slot), save :: g_models(NMODELS)
  type(kv_slot), save :: g_caches(NCACHES)
  ! the model and cache of the latest call (fgpt_handles, sample_next)
  type(c_ptr), save :: g_model = c_null_ptr
  type(c_ptr), save :: g_kv = c_null_ptr
  integer, save :: g_imodel = 0
  ! fgpt_forward_f16: applied to every bound model and to those bound later
  logical, save :: g_fwd_f16 = .false.

contains

  subroutine die(what, rc)
    character(*), intent(in) :: what
    integer(c_int32_t), intent(in) :: rc
    write (error_unit, '(4A,I0,A)') what, ': ', fg_error_message(), ' (rc ', rc, ')'
    error stop 1
  end subroutine die

  ! Bind the engine model of these weight arrays and dims (uploaded on
  ! first use); it becomes g_model.
  subroutine bind_model(wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, &
      vocab_size, d_model, n_head, n_kv_head, head_dim, n_layer, eps)
    real(c_float), intent(in), target :: wte(:), c_q(:), c_k(:), c_v(:), c_proj(:), &
        c_fc(:), c_proj2(:), lm_head(:)
    integer(c_int), intent(in) :: vocab_size, d_model, n_head, n_kv_head, head_dim, n_layer
    real(c_float), intent(in) :: eps
    integer(c_intptr_t) :: key(8)
    integer :: dims(6), i, free
    type(fg_dims) :: fd
    integer(c_int32_t) :: rc

    key = [transfer(c_loc(wte), 0_c_intptr_t), transfer(c_loc(c_q), 0_c_intptr_t), &
        transfer(c_loc(c_k), 0_c_intptr_t), transfer(c_loc(c_v), 0_c_intptr_t), &
        transfer(c_loc(c_proj), 0_c_intptr_t), transfer(c_loc(c_fc), 0_c_intptr_t), &
        transfer(c_loc(c_proj2), 0_c_intptr_t), transfer(c_loc(lm_head), 0_c_intptr_t)]
    dims = [n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size]
    free = 0
    do i = 1, NMODELS
      if (c_associated(g_models(i)%h)) then
        if (all(g_models(i)%key == key) .and. all(g_models(i)%dims == dims) .and. &
            g_models(i)%eps == eps) then
          g_imodel = i
          g_model = g_models(i)%h
          return
        end if
      else if (free == 0) then
        free = i
      end if
    end do
    if (free == 0) then
      write (error_unit, '(A,I0,A)') 'fgpt: more than ', NMODELS, &
          ' distinct weight sets or depths in use (call fgpt_release())'
      error stop 1
    end if
    if (size(wte) < vocab_size*d_model .or. size(lm_head) < vocab_size*d_model .or. &
        size(c_q) < n_layer*n_head*head_dim*d_model .or. &
        size(c_k) < n_layer*n_kv_head*head_dim*d_model .or. &
        size(c_v) < n_layer*n_kv_head*head_dim*d_model .or. &
        size(c_proj) < n_layer*d_model*n_head*head_dim .or. &
        size(c_fc) < n_layer*4*d_model*d_model .or. size(c_proj2) < n_layer*4*d_model*d_model) then
      write (error_unit, '(A)') 'fgpt: weight arrays smaller than the dims require'
      error stop 1
    end if
    fd = fg_dims(n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size, eps)
    rc = fg_model_create(fd, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, g_models(free)%h)
    if (rc /= FG_OK) call die('fgpt: weight upload', rc)
    g_models(free)%key = key
    g_models(free)%dims = dims
    g_models(free)%eps = eps
    g_imodel = free
    g_model = g_models(free)%h
    if (g_fwd_f16) then
      rc = fg_set_option(g_model, FG_OPT_FORWARD_F16, 1_c_int32_t)
      if (rc /= FG_OK) call die('fgpt: forward_f16', rc)
    end if
  end subroutine bind_model

  ! Single-term fp16 gpt_forward passes (see the header) on or off, for the
  ! models bound now and later.
  subroutine fgpt_forward_f16(on)
    logical, intent(in) :: on
    integer(c_int32_t) :: rc, v
    integer :: i
    g_fwd_f16 = on
    v = merge(1_c_int32_t, 0_c_int32_t, on)
    do i = 1, NMODELS
      if (c_associated(g_models(i)%h)) then
        rc = fg_set_option(g_models(i)%h, FG_OPT_FORWARD_F16, v)
        if (rc /= FG_OK) call die('fgpt: forward_f16', rc)
      end if
    end do
  end subroutine fgpt_forward_f16

  ! Bind the device cache of the caller's cache (its address) for the
  ! current model, B sequences of maxt positions; it becomes g_kv.
  subroutine bind_kv(cache_k, bb, maxt)
    real(c_float), intent(in), target :: cache_k(:)
    integer(c_int), intent(in) :: bb, maxt
    integer(c_intptr_t) :: addr
    integer :: i, free
    integer(c_int32_t) :: rc

    addr = transfer(c_loc(cache_k), 0_c_intptr_t)
    free = 0
    do i = 1, NCACHES
      if (c_associated(g_caches(i)%h)) then
        if (g_caches(i)%cache == addr .and. g_caches(i)%model == g_imodel .and. &
            g_caches(i)%bb == bb .and. g_caches(i)%maxt == maxt) then
          g_kv = g_caches(i)%h
          return
        end if
      else if (free == 0) then
        free = i
      end if
    end do
    if (free == 0) then
      write (error_unit, '(A,I0,A)') 'fgpt: more than ', NCACHES, &
          ' distinct caches in use (call fgpt_release())'
      error stop 1
    end if
    rc = fg_kv_create(g_model, bb, maxt, g_caches(free)%h)
    if (rc /= FG_OK) call die('fgpt: KV cache', rc)
    g_caches(free)%cache = addr
    g_caches(free)%model = g_imodel
    g_caches(free)%bb = bb
    g_caches(free)%maxt = maxt
    g_kv = g_caches(free)%h
  end subroutine bind_kv

  ! Drop every device model and cache (the next call uploads again).
  subroutine fgpt_release()
    integer(c_int32_t) :: rc
    integer :: i
    do i = 1, NCACHES
      if (c_associated(g_caches(i)%h)) rc = fg_kv_destroy(g_caches(i)%h)
      g_caches(i) = kv_slot()
    end do
    do i = 1, NMODELS
      if (c_associated(g_models(i)%h)) rc = fg_model_destroy(g_models(i)%h)
      g_models(i) = model_slot()
    end do
    g_kv = c_null_ptr
    g_model = c_null_ptr
    g_imodel = 0
  end subroutine fgpt_release

  ! The engine handles behind the drop-in calls (for callers that also use
  ! the C API directly, e.g. the device-side greedy loop).
  subroutine fgpt_handles(model, kv)
    type(c_ptr), intent(out) :: model, kv
    model = g_model
    kv = g_kv
  end subroutine fgpt_handles

  ! src/lib/fortran_gpt.f90:54-199. attn_blas selects another summation
  ! order of the same attention in the reference (attn_sgemm); here there is
  ! one attention kernel, so attn_blas changes no result. With attn_blas the
  ! reference also accumulates its positive-score statistic into pos_frac /
  ! pos_n (src/lib/fortran_attn.f90:247-300): per layer, row and head, the
  ! count of causal scores > 0 over T(T+1)/2, added in (layer, row) order;
  ! without attn_blas they are left alone, as the reference's causal_attn
  ! leaves them. attn_qk (QK-hop) is not part of this path and stops it.
  subroutine gpt_forward(idx, cos_buf, sin_buf, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, &
      lm_head, outp, BB, TT, vocab_size, d_model, n_head, n_kv_head, head_dim, n_layer, eps, &
      attn_blas, attn_qk, pos_frac, pos_n)
    integer(c_int), intent(in) :: BB, TT, vocab_size, d_model
    integer(c_int), intent(in) :: n_head, n_kv_head, head_dim, n_layer
    real(c_float), value :: eps
    logical, intent(in), optional :: attn_blas, attn_qk
    real(c_float), intent(inout), optional :: pos_frac(:)
    integer, intent(inout), optional :: pos_n(:)
    integer(c_int), intent(in) :: idx(:)
    real(c_float), intent(in) :: cos_buf(:), sin_buf(:)
    real(c_float), intent(in), target :: wte(:), c_q(:), c_k(:), c_v(:), c_proj(:), c_fc(:), &
        c_proj2(:), lm_head(:)
    real(c_float), intent(out) :: outp(:)
    integer(c_int32_t) :: rc
    logical :: stats
    integer(c_int32_t), allocatable :: npos(:)
    integer :: il, ib, ih

    if (present(attn_qk)) then
      if (attn_qk) then
        write (error_unit, '(A)') 'gpt_forward: attn_qk (QK-hop) is not supported by this engine'
        error stop 1
      end if
    end if
    stats = .false.
    if (present(attn_blas)) stats = attn_blas .and. present(pos_frac)
    if (stats) then
      if (size(pos_frac) < n_head) then
        write (error_unit, '(A)') 'gpt_forward: pos_frac smaller than n_head'
        error stop 1
      end if
      if (present(pos_n)) then
        if (size(pos_n) < n_head) then
          write (error_unit, '(A)') 'gpt_forward: pos_n smaller than n_head'
          error stop 1
        end if
      end if
    end if
    if (size(outp) < BB*TT*vocab_size .or. size(idx) < BB*TT .or. &
        size(cos_buf) < TT*(head_dim/2) .or. size(sin_buf) < TT*(head_dim/2)) then
      write (error_unit, '(A)') 'gpt_forward: array smaller than B*T requires'
      error stop 1
    end if
    call bind_model(wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, vocab_size, d_model, &
        n_head, n_kv_head, head_dim, n_layer, eps)
    rc = fg_set_rope(g_model, 0_c_int32_t, TT, cos_buf, sin_buf)
    if (rc /= FG_OK) call die('gpt_forward: RoPE tables', rc)
    if (.not. stats) then
      rc = fg_forward(g_model, idx, BB, TT, outp, c_null_ptr, c_null_ptr)
      if (rc /= FG_OK) call die('gpt_forward', rc)
      return
    end if
    allocate (npos(n_layer*BB*n_head))
    rc = fg_forward_pos(g_model, idx, BB, TT, outp, c_null_ptr, c_null_ptr, npos)
    if (rc /= FG_OK) call die('gpt_forward', rc)
    ! the reference's order: layers (gpt_forward), then rows and heads
    ! (attn_sgemm), one addition per (layer, row, head)
    do il = 1, n_layer
      do ib = 1, BB
        do ih = 1, n_head
          pos_frac(ih) = pos_frac(ih) + real(npos(((il-1)*BB + (ib-1))*n_head + ih), c_float) &
              / real(TT*(TT + 1)/2, c_float)
          if (present(pos_n)) pos_n(ih) = pos_n(ih) + 1
        end do
      end do
    end do
  end subroutine gpt_forward

  ! src/lib/fortran_kv.f90:26-149
  subroutine gpt_step(idx1, cos1, sin1, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, &
      cache_k, cache_v, cache_len, maxT, out1, BB, vocab_size, d_model, n_head, n_kv_head, &
      head_dim, n_layer, eps)
    integer(c_int), intent(in) :: BB, vocab_size, d_model
    integer(c_int), intent(in) :: n_head, n_kv_head, head_dim, n_layer
    integer(c_int), intent(in) :: maxT
    integer(c_int), intent(inout) :: cache_len
    real(c_float), value :: eps
    integer(c_int), intent(in) :: idx1(:)
    real(c_float), intent(in) :: cos1(:), sin1(:)
    real(c_float), intent(in), target :: wte(:), c_q(:), c_k(:), c_v(:), c_proj(:), c_fc(:), &
        c_proj2(:), lm_head(:)
    real(c_float), intent(inout), target :: cache_k(:), cache_v(:)
    real(c_float), intent(out) :: out1(:)
    integer(c_int32_t) :: rc

    if (cache_len >= maxT) then
      print '(A)', "gpt_step: cache full (raise maxT)"
      error stop 1
    end if
    call bind_model(wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, vocab_size, d_model, &
        n_head, n_kv_head, head_dim, n_layer, eps)
    call bind_kv(cache_k, BB, maxT)
    rc = fg_kv_set_len(g_kv, cache_len)
    if (rc /= FG_OK) call die('gpt_step', rc)
    rc = fg_set_rope(g_model, cache_len, 1_c_int32_t, cos1, sin1)
    if (rc /= FG_OK) call die('gpt_step: RoPE row', rc)
    rc = fg_step(g_model, g_kv, idx1, out1, c_null_ptr)
    if (rc /= FG_OK) call die('gpt_step', rc)
    cache_len = cache_len + 1
  end subroutine gpt_step

  ! src/lib/fortran_kv.f90:160-289
  subroutine gpt_step_multi(idx, cos_buf, sin_buf, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, &
      lm_head, cache_k, cache_v, cache_len, maxT, out, BB, vocab_size, d_model, n_head, &
      n_kv_head, head_dim, n_layer, TB, eps)
    integer(c_int), intent(in) :: BB, vocab_size, d_model
    integer(c_int), intent(in) :: n_head, n_kv_head, head_dim, n_layer
    integer(c_int), intent(in) :: maxT, TB
    integer(c_int), intent(inout) :: cache_len
    real(c_float), value :: eps
    integer(c_int), intent(in) :: idx(:)
    real(c_float), intent(in) :: cos_buf(:), sin_buf(:)
    real(c_float), intent(in), target :: wte(:), c_q(:), c_k(:), c_v(:), c_proj(:), c_fc(:), &
        c_proj2(:), lm_head(:)
    real(c_float), intent(inout), target :: cache_k(:), cache_v(:)
    real(c_float), intent(out) :: out(:)
    integer(c_int32_t) :: rc

    if (TB < 1) then
      print '(A)', "gpt_step_multi: TB must be >= 1"
      error stop 1
    end if
    if (cache_len + TB > maxT) then
      print '(A)', "gpt_step_multi: cache full (raise maxT)"
      error stop 1
    end if
    call bind_model(wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, vocab_size, d_model, &
        n_head, n_kv_head, head_dim, n_layer, eps)
    call bind_kv(cache_k, BB, maxT)
    rc = fg_kv_set_len(g_kv, cache_len)
    if (rc /= FG_OK) call die('gpt_step_multi', rc)
    rc = fg_set_rope(g_model, cache_len, TB, cos_buf, sin_buf)
    if (rc /= FG_OK) call die('gpt_step_multi: RoPE rows', rc)
    rc = fg_step_multi(g_model, g_kv, idx, TB, out, c_null_ptr)
    if (rc /= FG_OK) call die('gpt_step_multi', rc)
    cache_len = cache_len + TB
  end subroutine gpt_step_multi

  ! ------------------------------------------------------------ weights
  ! load_gpt_weights (src/lib/load_weights.f90:830-874): model.safetensors
  ! when the directory has one (canonical names, arch.* metadata checked),
  ! else the 1-D '<f4' .npy files with arch.txt checked when present. The
  ! engine's host reader does both; any failure stops the program with its
  ! message, as the reference's die/error stop do.
  subroutine load_gpt_weights(wdir, n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size, &
      wte, lm_head, c_q, c_k, c_v, c_pr, c_fc, c_pr2)
    character(*), intent(in) :: wdir
    integer, intent(in) :: n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size
    real(c_float), allocatable, intent(out) :: wte(:), lm_head(:)
    real(c_float), allocatable, intent(out) :: c_q(:), c_k(:), c_v(:), c_pr(:), c_fc(:), c_pr2(:)
    integer :: qsz, ksz, psz, fsz
    integer(c_int32_t) :: rc
    type(fg_dims) :: fd

    qsz = n_head*head_dim*d_model
    ksz = n_kv_head*head_dim*d_model
    psz = d_model*n_head*head_dim
    fsz = 4*d_model*d_model
    allocate (wte(vocab_size*d_model), lm_head(vocab_size*d_model))
    allocate (c_q(n_layer*qsz), c_k(n_layer*ksz), c_v(n_layer*ksz), c_pr(n_layer*psz))
    allocate (c_fc(n_layer*fsz), c_pr2(n_layer*fsz))
    fd = fg_dims(n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size, 1.0e-5_c_float)
    rc = fg_weights_read(fd, trim(wdir)//c_null_char, wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, &
        lm_head)
    if (rc /= FG_OK) call die('load_gpt_weights', rc)
  end subroutine load_gpt_weights

  ! accept_prefix (src/lib/fortran_spec.f90:41-52): the greedy accept rule,
  ! on the engine's host implementation. targmax holds k+1 ids.
  subroutine accept_prefix(draft, targmax, k, n_accept, correction)
    integer, intent(in) :: draft(:), targmax(:), k
    integer, intent(out) :: n_accept, correction
    integer(c_int32_t) :: d(max(k, 1)), t(k + 1), na, corr, rc

    if (k > 0) d(1:k) = int(draft(1:k), c_int32_t)
    t = int(targmax(1:k + 1), c_int32_t)
    rc = fg_spec_accept(d, t, int(k, c_int32_t), na, corr)
    if (rc /= FG_OK) call die('fg_spec_accept', rc)
    n_accept = na
    correction = corr
  end subroutine accept_prefix

  ! lookup_draft (src/lib/fortran_spec.f90:62-92): prompt-lookup proposals
  ! over ids(1:p), on the engine's host implementation.
  subroutine lookup_draft(ids, p, m, k, d, kk)
    integer, intent(in) :: ids(:), p, m, k
    integer, intent(out) :: d(:), kk
    integer(c_int32_t) :: x(max(p, 1)), o(max(k, 1)), n, rc

    if (p > 0) x(1:p) = int(ids(1:p), c_int32_t)
    rc = fg_spec_draft(x, int(p, c_int32_t), int(m, c_int32_t), int(k, c_int32_t), o, n)
    if (rc /= FG_OK) call die('fg_spec_draft', rc)
    kk = n
    if (kk > 0) d(1:kk) = o(1:kk)
  end subroutine lookup_draft

  ! sample_next (src/lib/sample.f90:153-177): the 1-based position of the
  ! sampled token, drawn on the device of the bound model (the model a
  ! gpt_forward / gpt_step / gpt_step_multi call has bound). state is the
  ! caller's xorshift64* state, advanced as the reference advances it.
  integer function sample_next(logits, V, temp, topp, pres, freq, rep, pwin, plen, gen, ngen, &
      nblock, state, byte_space)
    integer, intent(in) :: V, ngen, nblock, pwin
    real(c_float), intent(in) :: logits(:), temp, topp, pres, freq, rep, plen
    integer, intent(in) :: gen(:)
    integer(c_int64_t), intent(inout) :: state
    logical, intent(in), optional :: byte_space
    type(fg_sample_cfg) :: cfg
    integer(c_int32_t) :: g(max(ngen, 1)), id, rc

    if (.not. c_associated(g_model)) then
      write (error_unit, '(A)') 'sample_next: no model bound (call gpt_step or gpt_forward first)'
      error stop 1
    end if
    cfg = fg_sample_cfg(temp, topp, pres, freq, rep, plen, int(pwin, c_int32_t), &
        int(nblock, c_int32_t), 0_c_int32_t)
    if (present(byte_space)) then
      if (byte_space) cfg%byte_space = 1
    end if
    if (ngen > 0) g(1:ngen) = int(gen(1:ngen), c_int32_t)
    rc = fg_sample(g_model, logits, int(V, c_int32_t), g, int(ngen, c_int32_t), cfg, state, id)
    if (rc /= FG_OK) call die('fg_sample', rc)
    sample_next = id + 1
  end function sample_next

end module fgpt_drop_in_mod
