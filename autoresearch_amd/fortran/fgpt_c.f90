! fgpt_c.f90 -- iso_c_binding interface to the gfx950 engine (include/fgpt.h).
!
! The binding style is the reference's own for its rocBLAS shim
! (src/lib/fortran_blas_gpu.f90:30-59 binding src/lib/gpu_shim.cpp:98-122):
! plain bind(C) interfaces, integer return codes, pointers passed as
! assumed-size arrays or type(c_ptr).
module fgpt_c
  use, intrinsic :: iso_c_binding
  implicit none
  private

  integer(c_int32_t), parameter, public :: FG_OK = 0, FG_EARG = -1, FG_EDIMS = -2, &
      FG_EWEIGHT = -3, FG_EHIP = -4, FG_EFULL = -5, FG_EROPE = -6, FG_ENODEV = -7, &
      FG_EBUSY = -8, FG_EARCH = -9, FG_ERANGE = -10
  integer(c_int32_t), parameter, public :: FG_OPT_FUSED_DECODE = 1, FG_OPT_FORWARD_F16 = 2

  type, bind(C), public :: fg_dims
    integer(c_int32_t) :: n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size
    real(c_float) :: eps
  end type fg_dims

  ! --spec, --match, --spec-probe, --spec-min-acc (src/app/chat_text.f90:117-120)
  type, bind(C), public :: fg_spec_cfg
    integer(c_int32_t) :: k, match, probe
    real(c_float) :: min_acc
  end type fg_spec_cfg

  type, bind(C), public :: fg_spec_stats
    integer(c_int64_t) :: passes, accepted, proposed, plain, pauses
  end type fg_spec_stats

  ! --temp --topp --pres --freq --rep --plen --pwin --nblock --space byte
  ! (src/app/chat_text.f90:118-128)
  type, bind(C), public :: fg_sample_cfg
    real(c_float) :: temp, topp, pres, freq, rep, plen
    integer(c_int32_t) :: pwin, nblock, byte_space
  end type fg_sample_cfg

  public :: fg_version, fg_last_error, fg_model_create, fg_weights_read, fg_model_load, &
      fg_model_destroy, &
      fg_set_rope, fg_forward, fg_forward_pos, fg_kv_create, fg_kv_destroy, fg_kv_len, fg_kv_set_len, &
      fg_step, fg_step_multi, fg_decode_greedy, fg_sync, fg_eval_bpb, fg_rows_npy, &
      fg_decode_spec, fg_spec_accept, fg_spec_draft, fg_sample, fg_decode_sample, fg_set_option, &
      fg_error_message

  interface
    integer(c_int32_t) function fg_version() bind(C, name="fg_version")
      import :: c_int32_t
    end function

    integer(c_int32_t) function fg_last_error(buf, len) bind(C, name="fg_last_error")
      import :: c_int32_t, c_char
      character(kind=c_char), intent(out) :: buf(*)
      integer(c_int32_t), value :: len
    end function

    integer(c_int32_t) function fg_model_create(dims, wte, c_q, c_k, c_v, c_proj, c_fc, &
        c_proj2, lm_head, out) bind(C, name="fg_model_create")
      import :: c_int32_t, c_float, c_ptr, fg_dims
      type(fg_dims), intent(in) :: dims
      real(c_float), intent(in) :: wte(*), c_q(*), c_k(*), c_v(*), c_proj(*), c_fc(*), &
          c_proj2(*), lm_head(*)
      type(c_ptr), intent(out) :: out
    end function

    integer(c_int32_t) function fg_weights_read(dims, weights_dir, wte, c_q, c_k, c_v, &
        c_proj, c_fc, c_proj2, lm_head) bind(C, name="fg_weights_read")
      import :: c_int32_t, c_char, c_float, fg_dims
      type(fg_dims), intent(in) :: dims
      character(kind=c_char), intent(in) :: weights_dir(*)
      real(c_float), intent(out) :: wte(*), c_q(*), c_k(*), c_v(*), c_proj(*), c_fc(*), &
          c_proj2(*), lm_head(*)
    end function

    integer(c_int32_t) function fg_eval_bpb(m, rows, n_rows, T, batch, token_bytes, &
        n_token_bytes, nll, row_nats, row_bytes, total_nats, total_bytes) &
        bind(C, name="fg_eval_bpb")
      import :: c_int32_t, c_int64_t, c_float, c_double, c_ptr
      type(c_ptr), value :: m
      integer(c_int32_t), intent(in) :: rows(*), token_bytes(*)
      integer(c_int32_t), value :: n_rows, T, batch, n_token_bytes
      real(c_float), intent(out) :: nll(*)
      real(c_double), intent(out) :: row_nats(*), total_nats
      integer(c_int64_t), intent(out) :: row_bytes(*), total_bytes
    end function

    integer(c_int32_t) function fg_rows_npy(path, n_rows, width, rows) bind(C, name="fg_rows_npy")
      import :: c_int32_t, c_char, c_ptr
      character(kind=c_char), intent(in) :: path(*)
      integer(c_int32_t), intent(out) :: n_rows, width
      type(c_ptr), value :: rows
    end function

    integer(c_int32_t) function fg_model_load(dims, weights_dir, out) &
        bind(C, name="fg_model_load")
      import :: c_int32_t, c_char, c_ptr, fg_dims
      type(fg_dims), intent(in) :: dims
      character(kind=c_char), intent(in) :: weights_dir(*)
      type(c_ptr), intent(out) :: out
    end function

    integer(c_int32_t) function fg_model_destroy(m) bind(C, name="fg_model_destroy")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: m
    end function

    integer(c_int32_t) function fg_set_rope(m, pos0, n_pos, cos_buf, sin_buf) &
        bind(C, name="fg_set_rope")
      import :: c_int32_t, c_float, c_ptr
      type(c_ptr), value :: m
      integer(c_int32_t), value :: pos0, n_pos
      real(c_float), intent(in) :: cos_buf(*), sin_buf(*)
    end function

    integer(c_int32_t) function fg_forward(m, ids, B, T, logits, targets, nll) &
        bind(C, name="fg_forward")
      import :: c_int32_t, c_float, c_ptr
      type(c_ptr), value :: m
      integer(c_int32_t), intent(in) :: ids(*)
      integer(c_int32_t), value :: B, T
      real(c_float), intent(out) :: logits(*)
      type(c_ptr), value :: targets, nll
    end function

    ! fg_forward with attn_sgemm's positive-score counts, npos(n_layer*B*n_head)
    integer(c_int32_t) function fg_forward_pos(m, ids, B, T, logits, targets, nll, npos) &
        bind(C, name="fg_forward_pos")
      import :: c_int32_t, c_float, c_ptr
      type(c_ptr), value :: m
      integer(c_int32_t), intent(in) :: ids(*)
      integer(c_int32_t), value :: B, T
      real(c_float), intent(out) :: logits(*)
      type(c_ptr), value :: targets, nll
      integer(c_int32_t), intent(out) :: npos(*)
    end function

    integer(c_int32_t) function fg_kv_create(m, B, maxT, out) bind(C, name="fg_kv_create")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: m
      integer(c_int32_t), value :: B, maxT
      type(c_ptr), intent(out) :: out
    end function

    integer(c_int32_t) function fg_kv_destroy(kv) bind(C, name="fg_kv_destroy")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: kv
    end function

    integer(c_int32_t) function fg_kv_len(kv, len) bind(C, name="fg_kv_len")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: kv
      integer(c_int32_t), intent(out) :: len
    end function

    integer(c_int32_t) function fg_kv_set_len(kv, len) bind(C, name="fg_kv_set_len")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: kv
      integer(c_int32_t), value :: len
    end function

    integer(c_int32_t) function fg_step(m, kv, ids, logits, next_ids) bind(C, name="fg_step")
      import :: c_int32_t, c_float, c_ptr
      type(c_ptr), value :: m, kv
      integer(c_int32_t), intent(in) :: ids(*)
      real(c_float), intent(out) :: logits(*)
      type(c_ptr), value :: next_ids
    end function

    integer(c_int32_t) function fg_step_multi(m, kv, ids, TB, logits, next_ids) &
        bind(C, name="fg_step_multi")
      import :: c_int32_t, c_float, c_ptr
      type(c_ptr), value :: m, kv
      integer(c_int32_t), intent(in) :: ids(*)
      integer(c_int32_t), value :: TB
      real(c_float), intent(out) :: logits(*)
      type(c_ptr), value :: next_ids
    end function

    integer(c_int32_t) function fg_decode_spec(m, kv, ids, n_known, n_total, cfg, stats) &
        bind(C, name="fg_decode_spec")
      import :: c_int32_t, c_ptr, fg_spec_cfg, fg_spec_stats
      type(c_ptr), value :: m, kv
      integer(c_int32_t), intent(inout) :: ids(*)
      integer(c_int32_t), value :: n_known, n_total
      type(fg_spec_cfg), intent(in) :: cfg
      type(fg_spec_stats), intent(out) :: stats
    end function

    integer(c_int32_t) function fg_sample(m, logits, V, gen, ngen, cfg, state, id) &
        bind(C, name="fg_sample")
      import :: c_int32_t, c_int64_t, c_float, c_ptr, fg_sample_cfg
      type(c_ptr), value :: m
      real(c_float), intent(in) :: logits(*)
      integer(c_int32_t), value :: V, ngen
      integer(c_int32_t), intent(in) :: gen(*)
      type(fg_sample_cfg), intent(in) :: cfg
      integer(c_int64_t), intent(inout) :: state
      integer(c_int32_t), intent(out) :: id
    end function

    integer(c_int32_t) function fg_decode_sample(m, kv, ids, n_known, n_total, cfg, state) &
        bind(C, name="fg_decode_sample")
      import :: c_int32_t, c_int64_t, c_ptr, fg_sample_cfg
      type(c_ptr), value :: m, kv
      integer(c_int32_t), intent(inout) :: ids(*)
      integer(c_int32_t), value :: n_known, n_total
      type(fg_sample_cfg), intent(in) :: cfg
      integer(c_int64_t), intent(inout) :: state
    end function

    integer(c_int32_t) function fg_spec_accept(draft, targmax, k, n_accept, correction) &
        bind(C, name="fg_spec_accept")
      import :: c_int32_t
      integer(c_int32_t), intent(in) :: draft(*), targmax(*)
      integer(c_int32_t), value :: k
      integer(c_int32_t), intent(out) :: n_accept, correction
    end function

    integer(c_int32_t) function fg_spec_draft(ids, p, m, k, draft, n_draft) &
        bind(C, name="fg_spec_draft")
      import :: c_int32_t
      integer(c_int32_t), intent(in) :: ids(*)
      integer(c_int32_t), value :: p, m, k
      integer(c_int32_t), intent(out) :: draft(*), n_draft
    end function

    integer(c_int32_t) function fg_decode_greedy(m, kv, ids, n_steps, ids_out, logits_out) &
        bind(C, name="fg_decode_greedy")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: m, kv
      integer(c_int32_t), intent(in) :: ids(*)
      integer(c_int32_t), value :: n_steps
      integer(c_int32_t), intent(out) :: ids_out(*)
      type(c_ptr), value :: logits_out
    end function

    integer(c_int32_t) function fg_sync(m) bind(C, name="fg_sync")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: m
    end function

    integer(c_int32_t) function fg_set_option(m, key, value) bind(C, name="fg_set_option")
      import :: c_int32_t, c_ptr
      type(c_ptr), value :: m
      integer(c_int32_t), value :: key, value
    end function
  end interface

contains

  ! The engine's message for the calling thread's last error.
  function fg_error_message() result(msg)
    character(len=:), allocatable :: msg
    character(kind=c_char) :: buf(512)
    integer(c_int32_t) :: rc
    integer :: i, n
    rc = fg_last_error(buf, 512_c_int32_t)
    n = 0
    do i = 1, 512
      if (buf(i) == c_null_char) exit
      n = i
    end do
    allocate (character(len=n) :: msg)
    do i = 1, n
      msg(i:i) = buf(i)
    end do
  end function fg_error_message

end module fgpt_c
